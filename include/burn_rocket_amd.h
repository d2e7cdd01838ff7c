/*
 * burn_rocket_amd.h — C ABI of the MI355X (gfx950) accelerator op surface.
 *
 * This is the boundary a Burn backend extension binds over FFI. It replaces the
 * `rocket-npu` driver calls that `crates/burn-rocket` makes today and keeps the
 * same op surface: resident fp16 weights and their matmul, resident W8A8 / GGUF
 * Q8_0 int8 weights and their matmul, masked grouped-query flash attention, and
 * the MoE expert pipeline. Each entry point cites the reference item it stands
 * in for (paths relative to the royalcat/burn-rocket tree).
 *
 * Conventions
 *   - Every entry returns RK_OK (0) or a negative status code with the meaning
 *     of `crates/rocket-npu/src/error.rs:11-51`; `rk_last_error()` returns the
 *     message of the last failure on the calling thread.
 *   - Calls are serialised by one engine mutex (`ext.rs:543-556`); work inside a
 *     call runs on the library's HIP stream (or the stream passed to a `_dev`
 *     entry) and is stream-ordered. Calls may use different streams: the
 *     library's internal scratch buffers are fenced with events, so a call
 *     that reuses one waits on the device for the last call that used it, and
 *     a buffer is only freed (grown, trimmed) after that use has completed.
 *   - Host entries (`rk_matmul`, `rk_attention`, ...) take and return host f32
 *     buffers, as Burn's flex tensors do; conversion to fp16 / int8 happens on
 *     the GPU. `_dev` entries take device pointers that are already resident in
 *     HBM and do no host<->device copies.
 *   - Weight handles are u64 ids that stay valid for the process lifetime
 *     (`ext.rs:39-43`).
 *   - Matrices are row-major. A weight is [N, K] (HF `[out, in]`), an activation
 *     is [M, K], the product is [M, N] = x · Wᵀ.
 */
#ifndef BURN_ROCKET_AMD_H
#define BURN_ROCKET_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: crates/rocket-npu/src/error.rs:11-51 ------------------ */
#define RK_OK 0
#define RK_E_SHAPE (-1)       /* unsupported shape or bad argument */
#define RK_E_TILING (-2)      /* shape not tileable (caller may fall back) */
#define RK_E_NOMEM (-3)       /* device or host allocation failed */
#define RK_E_DEVICE (-4)      /* HIP runtime / device failure */
#define RK_E_UNSUPPORTED (-5) /* feature not supported */
#define RK_E_RANGE (-6)       /* an fp16 value left its range (error.rs:22-24) */
#define RK_E_IO (-7)          /* I/O failure */

/* ---- weight kinds (ext.rs:1156-1161 `WeightKind`) ------------------------ */
#define RK_WEIGHT_F16 1 /* resident fp16 [N, K] */
#define RK_WEIGHT_I8 2  /* resident int8 codes [N, K] + f32 scales [N, K/group] */
#define RK_WEIGHT_QAT 3 /* resident per-channel int8 codes + w_scale [N] */

/* ---- attention mask modes (ext.rs:1643-1666 `MaskMode`) ------------------ *
 * With absolute query position t = q0 + i and key position j = k0 + jj:
 *   RK_MASK_NONE           every key visible
 *   RK_MASK_CAUSAL         j <= t
 *   RK_MASK_WINDOW         |t - j| <= window
 *   RK_MASK_CAUSAL_WINDOW  t - window < j <= t
 * q0 = k0 = 0 with n_q == n_kv is the full-sequence form; other offsets are the
 * query-chunk block forms (`masks.rs:44-114`). Masks are evaluated as
 * predicates inside the kernel; no mask tensor is built.                      */
#define RK_MASK_NONE 0
#define RK_MASK_CAUSAL 1
#define RK_MASK_WINDOW 2
#define RK_MASK_CAUSAL_WINDOW 3

/* Element types of the MLP glue ops (the f32 / f16 / bf16 inputs the
 * reference's glue accepts, ext.rs:1040-1050). */
#define RK_DTYPE_F32 0
#define RK_DTYPE_F16 1
#define RK_DTYPE_BF16 2

/* Glue of the fused gate|up GEMM (rk_matmul_w8a8_glu_dev). */
#define RK_GLU_SILU 1
#define RK_GLU_GELU 2

typedef uint64_t rk_weight_id;
typedef void *rk_stream; /* a hipStream_t; NULL selects the library stream */

/* ======================================================================== *
 * Engine                                                                    *
 * ======================================================================== */

/* Create the process-global engine on HIP device `device`. Later calls are
 * no-ops. Replaces `burn_rocket::init(threads)` (ext.rs:561-580). */
int rk_init(int device);

/* Message of the last failure on this thread ("" if none). Mirrors
 * `burn_rocket::Error`'s Display (lib.rs:125-140). */
const char *rk_last_error(void);

/* 1 when `rc` asks the caller to fall back to another path (RK_E_TILING),
 * as `burn_rocket::Error::is_fallback` (lib.rs:142-147). */
int rk_is_fallback(int rc);

/* Op time counters: `burn_rocket::stats()` / `stats_reset()` (ext.rs:165-200).
 * For the host-buffer entries device_s is the time of the op's kernels on the
 * device (events around each row chunk's kernels; the reference's T_NPU_US)
 * and convert_s the rest of the call's wall time: the host<->device copies
 * and waits that the kernels did not hide (its T_CONVERT_US). calls counts
 * matmul, attention and MoE calls, host-buffer and `_dev` alike; the `_dev`
 * entries return before their kernels finish and add no time. */
typedef struct {
  double convert_s;
  double device_s;
  uint64_t calls;
} rk_stats_t;
int rk_stats(rk_stats_t *out);
int rk_stats_reset(void);

/* Live memory held by the engine: `burn_rocket::mem_stats()` (ext.rs:206-252;
 * `MemStats`, lib.rs:44-84). The device scratch is per named buffer, grown to
 * the largest call that used it; attention_bytes is the part the attention
 * entries use (the reference's attention_bo_bytes, the rest its
 * matmul_bo_bytes); host_bytes is the page-locked staging of the host-buffer
 * entries (its *_host_bytes). */
typedef struct {
  uint64_t weights_bytes;   /* resident weights */
  uint64_t scratch_bytes;   /* device scratch, all buffers */
  uint64_t n_weights;
  uint64_t attention_bytes; /* device scratch of the attention entries */
  uint64_t host_bytes;      /* page-locked host staging */
  uint64_t n_scratch;       /* scratch buffers */
} rk_mem_stats_t;
int rk_mem_stats(rk_mem_stats_t *out);
/* Drop scratch above `budget` bytes / all scratch: `trim_scratch_to`,
 * `clear_scratch` (ext.rs:256-308). A zero budget also frees the page-locked
 * staging (allocated again by the next host-buffer call). */
int rk_trim_scratch_to(uint64_t budget);
int rk_clear_scratch(void);
/* `trim_scratch` (ext.rs:254-265): frees the scratch buffers that no call has
 * used since the previous rk_trim_scratch; what the calls in between used
 * stays, as the reference keeps the just-used shape set. */
int rk_trim_scratch(void);

/* ======================================================================== *
 * Resident weights                                                          *
 * ======================================================================== */

/* fp16 weight from f32 [N, K] (RNE), `pack` (ext.rs:1866, pack_one ext.rs:869,
 * to_host ext.rs:758-776). */
int rk_pack(const float *w, int64_t n, int64_t k, rk_weight_id *id);
/* fp16 weight from fp16 bits [N, K] (the F16 arm of to_host, ext.rs:770). */
int rk_pack_f16(const uint16_t *w, int64_t n, int64_t k, rk_weight_id *id);
/* Segmented fp16 weight: `nparts` f32 parts [ns[i], K] concatenated along N
 * (`pack2`/`pack3` → pack_seg, ext.rs:836-855, ext.rs:1870-1885). */
int rk_pack_seg(const float *const *parts, const int64_t *ns, int nparts,
                int64_t k, rk_weight_id *id);

/* Group-wise int8 weight from f32 [N, K]: per (n, K-group) scale
 * max(amax/127, 1e-12), codes round-half-away(x * (1/scale)) clamped to ±127
 * (`pack_i8` → quantize_i8_weight → quantize_row_groups, ext.rs:939-1012,
 * host.rs:77-90). group % 32 == 0 and K % group == 0. */
int rk_pack_i8(const float *w, int64_t n, int64_t k, int64_t group,
               rk_weight_id *id);
/* Pre-quantized group-wise weight: codes [N, K], scales [N, K/group]
 * (`RocketI8Ctx::pack_weight_gw`, lib.rs:363; int8.rs:458). scales may be
 * NULL: the codes alone, as `I8Context::pack_weight_gw` keeps them (the
 * scales then come with each rk_matmul_i8_gw call, int8.rs:644-676); group K
 * with NULL scales is the per-channel `I8Context::pack_weight` (int8.rs:452),
 * whose product is rk_matmul_i8. */
int rk_pack_i8_codes(const int8_t *codes, const float *scales, int64_t n,
                     int64_t k, int64_t group, rk_weight_id *id);
/* Replace the codes/scales of a resident group-wise weight in place
 * (`I8Context::rewrite_weight_gw`, int8.rs:521). NULL scales keep the
 * resident scales (the reference rewrites codes only, int8.rs:482-526). */
int rk_rewrite_i8(rk_weight_id id, const int8_t *codes, const float *scales);
/* GGUF Q8_0 weight: [N, K/32] blocks of 34 bytes {f16 d, int8 q[32]}
 * (src/util/gguf.rs:125-200), e.g. a pointer into an mmapped GGUF tensor. The
 * blocks cross PCIe once, as they are, and are split on the GPU into codes
 * [N, K] and f32(d) scales (exact, f16 subnormals included); group 32. */
int rk_pack_q8_0(const uint8_t *blocks, int64_t n, int64_t k, rk_weight_id *id);
/* GGUF Q8_0 weight quantized on the device from f32 [N, K] with llama.cpp's
 * rule (crates/rocket-npu/src/bin/q8_bench.rs:200-220): per 32 values
 * d = f16(amax/127), codes round-half-away(x / f32(d)) clamped to ±127.
 * K % 32 == 0. The resident form equals rk_pack_q8_0 of the same blocks. */
int rk_pack_q8_0_f32(const float *w, int64_t n, int64_t k, rk_weight_id *id);
/* Per-channel QAT weight (`pack_qat`, ext.rs:1382-1425): codes [N, K],
 * w_scale [N], static activation scale in_scale (0 = per-row dynamic
 * amax/127), output grid out_scale (0 = none). */
int rk_pack_qat(const int8_t *codes, const float *w_scale, int64_t n, int64_t k,
                float in_scale, float out_scale, rk_weight_id *id);

/* Kind (RK_WEIGHT_*), N, K and group of a resident weight. */
int rk_weight_info(rk_weight_id id, int *kind, int64_t *n, int64_t *k,
                   int64_t *group);

/* ======================================================================== *
 * Matmul                                                                    *
 * ======================================================================== */

/* Host-buffer entries (rk_matmul, rk_matmul_i8_gw, rk_matmul_i8, rk_attention,
 * rk_flash_attn_f16, rk_silu_mul, rk_gelu_mul, rk_rms_norm*, rk_rope) move
 * their buffers through page-locked staging slots (hipHostMalloc) with a
 * pool of CPU copy threads; row-separable ops run in row chunks so that the
 * upload of one chunk, the kernels of the previous one and the download of
 * the one before overlap. They return when the outputs are in host memory.
 *
 * Every matmul entry accepts M = 0 (an empty batch): the arguments are
 * checked as for any M, nothing is launched and RK_OK is returned, as the
 * reference's row-chunk loop (`while off < m`, ext.rs:1457) runs no chunk and
 * returns an empty [.., 0, N] tensor. */

/* y[M, N] = x[M, K] · Wᵀ for any resident weight, host f32 in and out
 * (`rocket_matmul` → matmul_impl, ext.rs:627, ext.rs:1208-1232):
 *   F16: x → fp16 (RNE), fp16 GEMM with f32 accumulation, fp16 result widened
 *        to f32 (matmul_f16, ext.rs:1437-1499);
 *   I8 : x quantized per row per weight group (quantize_i8_rows, ext.rs:1017),
 *        C = Σ_g (a_s[m,g]·w_s[n,g])·P_g with exact int32 P_g (matmul_i8,
 *        ext.rs:1505; detile_accum_i8_scaled, layout.rs:504-540);
 *   QAT: x quantized with the static scale (ties-to-even, [-128,127]) or per
 *        row dynamically, exact int32 C, epilogue acc·(in_scale·w_scale[n])
 *        and optional output-grid rounding (matmul_qat, ext.rs:1236-1373). */
int rk_matmul(rk_weight_id id, const float *x, int64_t m, int64_t k, float *y);

/* fp16 GEMM on host buffers (`RocketCtx::matmul_prepacked`, lib.rs:244-254;
 * Context::matmul_prepacked, context.rs:497-513): a fp16 [M, K], c fp16
 * [M, N], f32 accumulation. The reference's M % 4 padding
 * (lib.rs:500-511) is not needed: any M >= 0. */
int rk_matmul_f16(rk_weight_id id, const uint16_t *a, int64_t m, int64_t k, uint16_t *c);
/* `I8Context::matmul_gw` (int8.rs:644-676) on host buffers, as Clef's expert
 * workers call it (src/clef/engine_npu.rs:75-110): a int8 codes [M, K]
 * already quantized per row per group, a_scale [M, K/group], b_scale
 * [N, K/group] the weight scales of this call (NULL: those packed with the
 * weight); cf f32 [M, N] = Σ_g (a_scale[m,g]·b_scale[n,g])·P_g, groups
 * ascending, the product of each group's scales rounded first as the
 * reference does (int8.rs:663-667, src/clef/int8.rs:101-158). The weight is a
 * group-wise int8 weight. */
int rk_matmul_i8_gw(rk_weight_id id, const int8_t *a, const float *a_scale,
                    const float *b_scale, int64_t m, int64_t k, float *cf);
/* `I8Context::matmul` (int8.rs:606-640) on host buffers: c int32 [M, N] =
 * Σ_k a[m,k]·w[n,k], exact, for an int8 weight of any group. */
int rk_matmul_i8(rk_weight_id id, const int8_t *a, int64_t m, int64_t k, int32_t *c);

/* fp16 GEMM on device buffers: a fp16 [M, K], c fp16 [M, N]
 * (`RocketCtx::matmul_prepacked`, lib.rs:244-254). K % 8 == 0. */
int rk_matmul_f16_dev(rk_weight_id id, const void *a, int64_t m, int64_t k,
                      void *c, rk_stream stream);

/* A gated MLP's first projection as one fp16 GEMM with the glue in its
 * epilogue: out [M, n] = glue(gate·x, up·x), glue = silu_mul (RK_GLU_SILU) or
 * gelu_mul (RK_GLU_GELU). It fuses what the reference's Qwen3 MLP runs as one
 * fp16 matmul on the pack2 of gate and up, a slice into the two halves and a
 * glue op (src/qwen3_embedding/model.rs:592-600 with the weights of
 * load.rs:221-238; matmul_f16 ext.rs:1437-1499, whose fp16 output is widened
 * to f32; rocket_silu_mul / rocket_gelu_mul ext.rs:603-608 with the formulas
 * of host.rs:12-39): each product is accumulated in f32, rounded to fp16 as
 * the plain GEMM's output is, then the glue runs in f32 with no FMA
 * contraction. a fp16 [M, K]; out f32 or (out_f16) fp16 [M, n]. The weight
 * comes from rk_pack_f16_glu (f32 gate and up, each [n, K], rounded to fp16
 * and interleaved per 16 rows); such a weight is only accepted here. */
int rk_pack_f16_glu(const float *gate, const float *up, int64_t n, int64_t k, rk_weight_id *id);
int rk_matmul_f16_glu_dev(rk_weight_id id, const void *a, int64_t m, int64_t k, int glu, void *out,
                          int out_f16, rk_stream stream);

/* Per-row activation quantizer on device (`quantize_i8_rows`, ext.rs:1017;
 * quantize_row_groups, host.rs:77-90): x f32 [M, K] → q int8 [M, K] and
 * scale f32 [M, K/group]. group == K is per-token quantization. */
int rk_quantize_rows_dev(const float *x, int64_t m, int64_t k, int64_t group,
                         int8_t *q, float *scale, rk_stream stream);

/* W8A8 GEMM on device buffers against a resident I8 weight
 * (`I8Context::matmul_gw`, int8.rs:644-676): a int8 [M, K] with scales
 * a_scale [M, K/a_group]; a_group is the weight's group (the reference's
 * Σ_g (a_s·w_s)·P_g) or K (per-token: a_s[m]·Σ_g w_s[n,g]·P_g).
 * c f32 [M, N]. Groups are summed in ascending order in f32 with exact int32
 * P_g; the rounding inside each term is not the reference's two-step
 * acc + fl(fl(a_s·w_s)·P_g): weights whose every scale is an fp16 value (GGUF
 * Q8_0 d) fold fma(fl(P_g·d), a_s, acc), others fma(P_g, fl(a_s·w_s), acc).
 * Both stay within 1e-5 of the largest output against the reference formula
 * at the config-2 shapes. rk_matmul_i8_gw folds every weight the second way. */
int rk_matmul_w8a8_dev(rk_weight_id id, const int8_t *a, const float *a_scale,
                       int64_t a_group, int64_t m, int64_t k, float *c,
                       rk_stream stream);
/* Same, fp16 output. */
int rk_matmul_w8a8_f16out_dev(rk_weight_id id, const int8_t *a,
                              const float *a_scale, int64_t a_group, int64_t m,
                              int64_t k, void *c, rk_stream stream);

/* Raw integer product of int8 activations and a resident I8/QAT weight's
 * codes: c int32 [M, N] = Σ_k a[m,k]·w[n,k], exact (`I8Context::matmul`,
 * int8.rs:606-640). */
int rk_matmul_i8_raw_dev(rk_weight_id id, const int8_t *a, int64_t m, int64_t k,
                         int32_t *c, rk_stream stream);

/* Per-block int32 partials of the same product: p int32 [M, N, K/32],
 * p[m,n,b] = Σ_{k in block b} a[m,k]·w[n,k] over 32-value blocks. Exposes
 * the accumulators the scaled W8A8 kernel folds, for exactness checks (the
 * per-K-tile partials of `drain`, int8.rs:708-746). */
int rk_matmul_i8_partials_dev(rk_weight_id id, const int8_t *a, int64_t m,
                              int64_t k, int32_t *p, rk_stream stream);

/* ======================================================================== *
 * Attention                                                                 *
 * ======================================================================== */

/* Masked grouped-query attention, token-major host f32 buffers as Burn passes
 * them (`rocket_attention*` → attention_impl, ext.rs:631-755,
 * ext.rs:1669-1858): q [n_q, n_head·head_dim], k/v [n_kv, n_kv_heads·head_dim],
 * out [n_q, n_head·head_dim]. Query head h reads kv head h / (n_head /
 * n_kv_heads). Score = scale·q·k (softcap·tanh(score/softcap) when softcap !=
 * 0), f32 online softmax over the visible keys, fp16 operands, fp16 result
 * widened to f32. A query row with no visible key averages V uniformly over
 * the n_kv keys (flash_attn_ref, attn/oneshot.rs:118-127). window < 0 turns
 * the window modes into NONE / CAUSAL (ext.rs:99-126). head_dim: 32, 48, 64,
 * 72, 80, 96, 112, 128 or 256, and 160, 192, 224 (run zero-padded to 256, on
 * packed rows; the reference's contract is head_dim % 32, attn/mod.rs:1443);
 * others return RK_E_UNSUPPORTED. A q or k value that fp16 cannot represent
 * returns RK_E_RANGE (the reference answers Status::Range when its fp16 score
 * surface saturates, attn/softmax.rs:462-475; scores are f32 here). */
int rk_attention(const float *q, const float *k, const float *v, int64_t n_q,
                 int64_t n_kv, int n_head, int n_kv_heads, int head_dim,
                 float scale, float softcap, int mask_mode, int64_t window,
                 int64_t q0, int64_t k0, float *out);

/* The same on fp16 device buffers in the token-major layout. Library scratch
 * holds V transposed and, when the launch has at most half as many query
 * tiles as the GPU has CUs, the partial softmax states of query tiles whose
 * keys are split between two workgroups (merged in a fixed order: results are
 * the same from call to call). */
int rk_attention_dev(const void *q, const void *k, const void *v, int64_t n_q,
                     int64_t n_kv, int n_head, int n_kv_heads, int head_dim,
                     float scale, float softcap, int mask_mode, int64_t window,
                     int64_t q0, int64_t k0, void *out, rk_stream stream);
/* No counterpart in the reference: rk_attention_dev for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). It calls no allocating routine: the
 * V-transposed operand goes to a static device array of
 * RK_NOALLOC_SCRATCH_BYTES per GPU (held from rk_init until the process ends)
 * instead of library scratch. Shapes whose Vᵀ, n_kv_heads · dv_pad ·
 * round_up(n_kv, 64) · 2 bytes with dv_pad = head_dim rounded up to 16, is
 * larger return RK_E_NOMEM. All calls on one GPU share that array and each
 * call rewrites it: calls whose work overlaps on the device (different streams
 * with no ordering between them) race and give wrong results. It never
 * splits a query tile's keys (that needs a workspace), and it refuses head
 * dims 160, 192 and 224 with RK_E_UNSUPPORTED (rk_attention_dev runs those
 * zero-padded to 256 in scratch); otherwise the same arguments and results as
 * rk_attention_dev (bit for bit when that split is off, RK_ATTN_SPLIT=1). */
#define RK_NOALLOC_SCRATCH_BYTES (32u << 20)
int rk_attention_dev_noalloc(const void *q, const void *k, const void *v, int64_t n_q,
                             int64_t n_kv, int n_head, int n_kv_heads, int head_dim, float scale,
                             float softcap, int mask_mode, int64_t window, int64_t q0, int64_t k0,
                             void *out, rk_stream stream);
/* rk_attention_dev with token strides (in values; multiples of 8, buffers
 * 16-byte aligned): q, k, v and out may be column ranges of wider rows, e.g.
 * the q, k and v parts of one fused q|k|v projection output, read where they
 * lie (the reference slices them into separate tensors first,
 * src/qwen3_embedding/model.rs:355-368). */
int rk_attention_strided_dev(const void *q, int64_t q_stride, const void *k, int64_t k_stride,
                             const void *v, int64_t v_stride, int64_t n_q, int64_t n_kv,
                             int n_head, int n_kv_heads, int head_dim, float scale,
                             float softcap, int mask_mode, int64_t window, int64_t q0,
                             int64_t k0, void *out, int64_t out_stride, rk_stream stream);

/* Head-major fp16 host buffers, the `RocketFaCtx::flash_attn` layout
 * (lib.rs:294-323; attn/mod.rs:1541-1600; shape contract check_flash,
 * attn/mod.rs:1424-1460): q [n_head][n_q][head_dim], k [n_kv_heads][n_kv]
 * [head_dim], v transposed [n_kv_heads][dv][n_kv], out [n_head][n_q][dv].
 * head_dim (the q·k width) and dv (the v width) are independent, as in the
 * reference's padded calls (Clef's 72-wide vision heads as head_dim 96,
 * dv 80: src/clef/vision/npu.rs:211-230); max(head_dim, dv) is zero-padded
 * to the next kernel width (32, 48, 64, 72, 80, 96, 112, 128, 256), so the
 * reference's contract head_dim % 32, dv % 16 (attn/mod.rs:1443) holds up to
 * 256; wider heads return RK_E_UNSUPPORTED. The reference's optional
 * additive mask tensor is replaced by mask_mode / window / q0 / k0. */
int rk_flash_attn_f16(int64_t n_q, int64_t n_kv, int head_dim, int dv,
                      int n_head, int n_kv_heads, float scale, float softcap,
                      int mask_mode, int64_t window, int64_t q0, int64_t k0,
                      const uint16_t *q, const uint16_t *k, const uint16_t *v,
                      uint16_t *out);
/* `RocketFaCtx::flash_attn` (lib.rs:294-323; Attention::flash,
 * attn/mod.rs:1541-1600) with its optional additive mask: mask fp16
 * [n_q, n_kv] of 0 (visible) and -inf (hidden), or NULL for none. Masks of
 * the reference's builders (masks.rs:11-114: causal, band and causal window,
 * full-sequence or block forms) run as the kernel's predicates, found by one
 * pass over the mask on the host; any other mask (other values, or visible
 * keys that are not one interval per row, or rows that follow no one mode)
 * returns RK_E_UNSUPPORTED. Layouts and padding as rk_flash_attn_f16. */
int rk_flash_attn_f16_masked(int64_t n_q, int64_t n_kv, int head_dim, int dv, int n_head,
                             int n_kv_heads, float scale, float softcap, const uint16_t *mask,
                             const uint16_t *q, const uint16_t *k, const uint16_t *v, uint16_t *out);

/* ======================================================================== *
 * MoE experts                                                               *
 * ======================================================================== */

/* Router: softmax over n_experts logits per token, top_k descending with ties
 * to the lower id, optional renormalisation (`route`, src/clef/model.rs:462-489).
 * logits f32 [s, n_experts] → ids u32 [s, top_k], wts f32 [s, top_k]. Host. */
int rk_moe_route(const float *logits, int64_t s, int n_experts, int top_k,
                 int norm_topk, uint32_t *ids, float *wts);

/* Resident expert stack: n_experts Q8_0 expert FFNs, each gate [inter, hidden],
 * up [inter, hidden], down [hidden, inter], as GGUF Q8_0 blocks
 * (src/clef/engine_npu.rs:110-207 packs gate|up and down per expert). Each
 * expert's blocks are uploaded as they are and split on the GPU into the
 * fragment-major layout the expert kernels stream. */
int rk_pack_moe_q8_0(const uint8_t *gate, const uint8_t *up,
                     const uint8_t *down, int n_experts, int64_t hidden,
                     int64_t inter, rk_weight_id *id);

/* The same expert stack from f32 weights (gate/up [E][inter][hidden], down
 * [E][hidden][inter]), quantized to Q8_0 on the device as rk_pack_q8_0_f32. */
int rk_pack_moe_f32(const float *gate, const float *up, const float *down,
                    int n_experts, int64_t hidden, int64_t inter,
                    rk_weight_id *id);

/* Expert FFN over routed tokens on device buffers: per token t and slot j,
 * y[t] += wts[t,j] · down(silu(gate(x_t)) ⊙ up(x_t)) of expert ids[t,j], the
 * slots summed in ascending expert id (combine, src/clef/engine.rs:317-338;
 * layer_forward_multi, src/clef/model.rs:526-620), with the W8A8 arithmetic
 * of the reference's expert workers (EmuWorker::run, src/clef/engine.rs:
 * 990-1043; NpuWorker/gw_matmul, src/clef/engine_npu.rs:75-207): x f32
 * [s, hidden] and the silu·up rows are each quantized per row per 32-value
 * group (scale max(amax/127, 1e-12), round-half-away, ±127), and every
 * product is Σ_b (a_s[m,b]·w_s[n,b])·P_b over the Q8_0 blocks b with exact
 * int32 P_b, accumulated in f32 in ascending b. The gate|up product rounds
 * each term as the reference does, acc + fl(fl(a_s·w_s)·P_b) (its results are
 * quantized again); the down product folds fma(fl(P_b·w_s), a_s, acc), within
 * 1e-5 of the largest value of the reference's order. silu(v) = v / (1 + e^-v) (src/clef/model.rs:
 * 491-493). ids/wts are host arrays (bucketing runs on the host,
 * engine.rs:284-313); y f32 [s, hidden] is overwritten with the sum. The
 * combine runs inside the down-projection launch: the workgroup that
 * completes a token's top_k rows (an arrival count per token and column
 * slice) sums them in ascending expert id, so y does not depend on the
 * order the workgroups finish in. RK_E_SHAPE when s·hidden or
 * s·top_k·inter reaches 2^31, or s·top_k·hidden·4 bytes reaches 2^31. */
int rk_moe_experts_dev(rk_weight_id id, const float *x, int64_t s, int top_k,
                       const uint32_t *ids, const float *wts, float *y,
                       rk_stream stream);
/* The same, accumulating onto y: y[t] = ((y[t] + out_e0) + out_e1) + …
 * with e0 < e1 < … the token's experts, the reference's combine onto the
 * residual it already holds (`let mut y = hid; … *a += b`, src/clef/model.rs:
 * 606-614; combine, src/clef/engine.rs:317-338). x and y may be the same
 * buffer (x is read before y is written). */
int rk_moe_experts_acc_dev(rk_weight_id id, const float *x, int64_t s, int top_k,
                           const uint32_t *ids, const float *wts, float *y,
                           rk_stream stream);

/* The same split in two: bucket once (host), keep the per-expert row lists,
 * tiles and combine order on the device, then run the expert FFN for any x
 * with that routing. Calls that use a plan must finish before it is
 * destroyed (rk_moe_plan_destroy synchronises the library stream). */
int rk_moe_plan_create(rk_weight_id id, int64_t s, int top_k,
                       const uint32_t *ids, const float *wts, void **plan);
int rk_moe_experts_planned_dev(rk_weight_id id, const void *plan,
                               const float *x, float *y, rk_stream stream);
int rk_moe_experts_planned_acc_dev(rk_weight_id id, const void *plan,
                                   const float *x, float *y, rk_stream stream);
int rk_moe_plan_destroy(void *plan);
/* First stage alone, for exactness checks: act f32 [rows, inter] =
 * silu(gate·x)·(up·x) for every bucket row, rows ordered by expert id and,
 * within an expert, by token (the bucket order of engine.rs:292-305). */
int rk_moe_gate_up_dev(rk_weight_id id, const void *plan, const float *x,
                       float *act, rk_stream stream);

/* ======================================================================== *
 * MLP glue                                                                 *
 * ======================================================================== */
/* out = silu(a)·b = a·(1/(1 + exp(-a)))·b elementwise over n values
 * (`rocket_silu_mul`, ext.rs:72, 607-608, silu_mul_impl ext.rs:1076-1090,
 * formula host.rs:30-39): computed in f32, inputs and output of type dtype
 * (RK_DTYPE_*), the output rounded to nearest even. Device buffers; out may
 * be a or b. */
int rk_silu_mul_dev(const void *a, const void *b, void *out, int64_t n, int dtype,
                    rk_stream stream);
/* out = gelu_tanh(a)·b, gelu_tanh(x) = (x·(tanh((x + x·x·x·0.044715)·√(2/π)) + 1))·0.5
 * (`rocket_gelu_mul`, ext.rs:70, 603-604, gelu_mul_impl ext.rs:1057-1072,
 * formula host.rs:12-28). Same conventions as rk_silu_mul_dev. */
int rk_gelu_mul_dev(const void *a, const void *b, void *out, int64_t n, int dtype,
                    rk_stream stream);
/* Host-buffer forms on f32 arrays (synchronous). */
int rk_silu_mul(const float *a, const float *b, float *out, int64_t n);
int rk_gelu_mul(const float *a, const float *b, float *out, int64_t n);

/* A gated MLP's first projection in one W8A8 GEMM with the glue in its
 * epilogue: out [M, n] = glue(gate·x, up·x), glue = silu_mul (RK_GLU_SILU)
 * or gelu_mul (RK_GLU_GELU). It fuses what the reference runs as two
 * matmuls and a glue op (`matmul_impl` ext.rs:1184-1232 on the gate and up
 * weights, then `rocket_silu_mul` / `rocket_gelu_mul` ext.rs:603-608; the
 * glue formulas host.rs:12-39): the gate and up products are the per-token
 * W8A8 results of rk_matmul_w8a8_dev (a int8 [M, K] with one scale per row,
 * a_scale [M]), the glue is computed in f32 and out is f32 or fp16
 * (out_f16). The weight comes from rk_pack_q8_0_glu (GGUF Q8_0 blocks of the
 * gate and up matrices, each [n, K]) or rk_pack_q8_0_glu_f32 (f32 gate and
 * up, quantized to Q8_0 on the device); such a weight is only accepted here. */
int rk_pack_q8_0_glu(const uint8_t *gate_blocks, const uint8_t *up_blocks, int64_t n,
                     int64_t k, rk_weight_id *id);
int rk_pack_q8_0_glu_f32(const float *gate, const float *up, int64_t n, int64_t k,
                         rk_weight_id *id);
int rk_matmul_w8a8_glu_dev(rk_weight_id id, const int8_t *a, const float *a_scale, int64_t m,
                           int64_t k, int glu, void *out, int out_f16, rk_stream stream);

/* ======================================================================== *
 * Normalisation and rotary embedding                                       *
 * ======================================================================== */
/* Weighted RMSNorm over the last dim: for each of `rows` rows of d values,
 * out = x·inv·w with inv = 1/sqrt(Σx²/d + eps) (`rocket_rms_norm`,
 * ext.rs:75-76, 611-612, rms_norm_impl ext.rs:1093-1107, row formula
 * host.rs:40-56; eps is taken as f64 and used as f32 like the reference).
 * Computed in f32; x and out of type dtype, w [d] of type w_dtype
 * (RK_DTYPE_*), out rounded to nearest even. The sum of squares runs in a
 * fixed parallel order (deterministic; not the reference's left-to-right
 * order). Device buffers; out may be x. */
int rk_rms_norm_dev(const void *x, const void *w, int w_dtype, void *out, int64_t rows, int64_t d,
                    double eps, int dtype, rk_stream stream);
/* Scale-free RMSNorm, out = x·inv (`rocket_rms_norm_noscale`, ext.rs:78-80,
 * 613-615, rms_norm_noscale_impl ext.rs:1109-1123). As rk_rms_norm_dev. */
int rk_rms_norm_noscale_dev(const void *x, void *out, int64_t rows, int64_t d, double eps,
                            int dtype, rk_stream stream);
/* Rotate-half RoPE of x [b, s, h, d] (row-major, d even) with cos/sin tables
 * [s, d/2]: out[j] = x[j]·cos[j] − x[d/2+j]·sin[j], out[d/2+j] =
 * x[d/2+j]·cos[j] + x[j]·sin[j], table row = the token's position in s
 * (`rocket_rope`, ext.rs:82-84, 617-619, rope_impl ext.rs:1125-1152, row
 * formula host.rs:58-75). Computed in f32 with no fused multiply-add; x and
 * out of type dtype, the tables of type cs_dtype. Device buffers; out may
 * be x. */
int rk_rope_dev(const void *x, const void *cos, const void *sin, int cs_dtype, void *out,
                int64_t b, int64_t s, int64_t h, int64_t d, int dtype, rk_stream stream);
/* The attention prologue of a fused q|k|v projection, in place: for each of
 * s tokens (rows `row_stride` values apart) the n_q_heads q heads and the
 * n_kv_heads k heads at the start of the row get RMSNorm over head_dim with
 * q_norm_w / k_norm_w [head_dim] (eps as in rk_rms_norm_dev; the result
 * rounded to dtype), then rotate-half RoPE with cos/sin row t for token t.
 * The values after the k heads (V) are not touched. It is the composite the
 * Qwen3 layer runs on the fused projection (src/qwen3_embedding/model.rs:
 * 355-376: `q_norm`/`k_norm` through `burn_rocket::rms_norm` ext.rs:2112-2119,
 * then `burn_rocket::rope_apply` ext.rs:2130-2137 with `cos_rows(0, s)`), in
 * one pass. The norm weights have type dtype, or are both NULL (RoPE only);
 * cos/sin [s, head_dim/2] have type dtype or f32. RK_E_UNSUPPORTED when
 * head_dim / row_stride / alignment leave no vector width of at most 64
 * values per lane (fp16: head_dim <= 512 with head_dim/2 % 8 == 0). */
int rk_qk_norm_rope_dev(void *qkv, int64_t s, int64_t row_stride, int n_q_heads, int n_kv_heads,
                        int64_t head_dim, const void *q_norm_w, const void *k_norm_w, double eps,
                        const void *cos, const void *sin, int cs_dtype, int dtype,
                        rk_stream stream);
/* A whole self-attention block on an fp16 q|k|v projection output, in two
 * launches: rk_qk_norm_rope_dev's in-place prologue (its conventions; the
 * same launch also rewrites V into the attention kernel's operand layout),
 * then attention over the s tokens as rk_attention_strided_dev with q, k and
 * v read from the buffer (n_head q heads at column 0, n_kv_heads k heads at
 * n_head·head_dim, V after them) and out [s, out_stride]. The qkv buffer
 * holds the normalised, rotated q and k afterwards. It is the Qwen3 layer's
 * fused-projection path, src/qwen3_embedding/model.rs:355-376 followed by its
 * attention call (model.rs:449-463), with no intermediate tensors. */
int rk_attention_qkv_dev(void *qkv, int64_t s, int64_t row_stride, int n_head, int n_kv_heads,
                         int head_dim, const void *q_norm_w, const void *k_norm_w, double eps,
                         const void *cos, const void *sin, int cs_dtype, float scale,
                         float softcap, int mask_mode, int64_t window, int64_t q0, int64_t k0,
                         void *out, int64_t out_stride, rk_stream stream);
/* RMSNorm then per-token int8 quantization in one pass: the activation input
 * of a per-token W8A8 GEMM (rk_matmul_w8a8_dev with a_group = K) after a norm,
 * e.g. the Qwen3 MLP input (`post_attention_layernorm` through
 * `burn_rocket::rms_norm`, ext.rs:2112-2119). It is not the reference's own
 * I8 matmul input: that quantizes each row per weight group (ext.rs:1017-1029
 * with quantize_row_groups host.rs:77-90; 32 values for Q8_0 weights), which
 * rk_rms_norm_dev followed by rk_quantize_rows_dev with group 32 produces.
 * y = rk_rms_norm_dev's result in dtype
 * (w NULL: scale-free; else w_dtype must equal dtype), then q_scale[row] =
 * max(amax(y)/127, 1e-12) and q = round-half-away(y·(1/q_scale)) clamped to
 * ±127, q int8 [rows, d]. RK_E_UNSUPPORTED unless d·sizeof(dtype) is a
 * multiple of 16 and at most 8 KB and x and w are 16-byte aligned. */
int rk_rms_norm_quantize_dev(const void *x, const void *w, int w_dtype, int64_t rows, int64_t d,
                             double eps, int dtype, int8_t *q, float *q_scale, rk_stream stream);
/* Host-buffer forms on f32 arrays (synchronous). */
int rk_rms_norm(const float *x, const float *w, float *out, int64_t rows, int64_t d, double eps);
int rk_rms_norm_noscale(const float *x, float *out, int64_t rows, int64_t d, double eps);
int rk_rope(const float *x, const float *cos, const float *sin, float *out, int64_t b, int64_t s,
            int64_t h, int64_t d);

/* ======================================================================== *
 * Device plumbing for callers without their own HIP runtime bindings       *
 * ======================================================================== */
int rk_device_alloc(size_t bytes, void **ptr);
int rk_device_free(void *ptr);
int rk_memcpy_htod(void *dst, const void *src, size_t bytes);
int rk_memcpy_dtoh(void *dst, const void *src, size_t bytes);
/* Device-to-device copy, ordered on `stream` (NULL: the library stream). */
int rk_memcpy_dtod(void *dst, const void *src, size_t bytes, rk_stream stream);
int rk_memset_dev(void *dst, int value, size_t bytes);
/* y = x converted element by element between f32, fp16 and bf16 (RK_DTYPE_*),
 * rounded to nearest even: the host f32_to_f16_par / f16_to_f32_par passes
 * either side of every reference op (ext.rs:2144-2170), on device buffers.
 * x and y must not overlap unless they are the same buffer and the types
 * have the same size. */
int rk_cast_dev(const void *x, int x_dtype, void *y, int y_dtype, int64_t n, rk_stream stream);
int rk_stream_get(rk_stream *stream);    /* the library stream */
/* A new non-blocking HIP stream at the default priority, and its release
 * (after rk_stream_sync when work is pending on it). */
int rk_stream_create(rk_stream *stream);
int rk_stream_destroy(rk_stream stream);
int rk_stream_sync(rk_stream stream);
int rk_event_create(void **event);
int rk_event_destroy(void *event);
int rk_event_record(void *event, rk_stream stream);
int rk_event_elapsed_ms(void *start, void *stop, float *ms);
/* Device name, compute units and clock (kHz) of the engine's device. */
int rk_device_info(char *name, size_t name_len, int *cus, int *clock_khz);

#ifdef __cplusplus
}
#endif
#endif /* BURN_ROCKET_AMD_H */
