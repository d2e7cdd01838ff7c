//! Raw FFI and thin safe wrappers for `libburn_rocket_amd.so`, the MI355X (gfx950)
//! replacement of the `rocket-npu` driver under `crates/burn-rocket`.
//!
//! The `extern "C"` block mirrors `include/burn_rocket_amd.h` one to one (same
//! names, argument order and types); `build.rs` compiles the HIP sources for
//! gfx950 with hipcc and links the library. The wrappers below turn the status
//! codes (`crates/rocket-npu/src/error.rs:11-51`) into `Error { op, rc }`, the
//! shape of `burn_rocket::Error` (`crates/burn-rocket/src/lib.rs:119-156`).
//!
//! Not built in the repository that holds it (there is no Rust toolchain there);
//! `tests/test_rust_binding.py` checks the declarations against the header.

#![allow(non_camel_case_types)]

use std::ffi::CStr;
use std::os::raw::{c_char, c_int, c_void};

/// Registry id of a resident weight (`rk_weight_id`).
pub type WeightId = u64;
/// A `hipStream_t`; null selects the library stream.
pub type Stream = *mut c_void;

pub const RK_OK: c_int = 0;
pub const RK_E_SHAPE: c_int = -1;
pub const RK_E_TILING: c_int = -2;
pub const RK_E_NOMEM: c_int = -3;
pub const RK_E_DEVICE: c_int = -4;
pub const RK_E_UNSUPPORTED: c_int = -5;
pub const RK_E_RANGE: c_int = -6;
pub const RK_E_IO: c_int = -7;

pub const RK_WEIGHT_F16: c_int = 1;
pub const RK_WEIGHT_I8: c_int = 2;
pub const RK_WEIGHT_QAT: c_int = 3;

pub const RK_MASK_NONE: c_int = 0;
pub const RK_MASK_CAUSAL: c_int = 1;
pub const RK_MASK_WINDOW: c_int = 2;
pub const RK_MASK_CAUSAL_WINDOW: c_int = 3;

pub const RK_DTYPE_F32: c_int = 0;
pub const RK_DTYPE_F16: c_int = 1;
pub const RK_DTYPE_BF16: c_int = 2;

pub const RK_GLU_SILU: c_int = 1;
pub const RK_GLU_GELU: c_int = 2;

pub const RK_NOALLOC_SCRATCH_BYTES: usize = 32 << 20;

/// `rk_stats_t`: conversion / device seconds of the host-buffer ops and the call count.
#[repr(C)]
#[derive(Debug, Default, Clone, Copy)]
pub struct RkStats {
    pub convert_s: f64,
    pub device_s: f64,
    pub calls: u64,
}

/// `rk_mem_stats_t`: live resident-weight, device scratch (all / attention)
/// and page-locked staging bytes.
#[repr(C)]
#[derive(Debug, Default, Clone, Copy)]
pub struct RkMemStats {
    pub weights_bytes: u64,
    pub scratch_bytes: u64,
    pub n_weights: u64,
    pub attention_bytes: u64,
    pub host_bytes: u64,
    pub n_scratch: u64,
}

#[link(name = "burn_rocket_amd")]
unsafe extern "C" {
    pub fn rk_init(device: c_int) -> c_int;
    pub fn rk_last_error() -> *const c_char;
    pub fn rk_is_fallback(rc: c_int) -> c_int;
    pub fn rk_stats(out: *mut RkStats) -> c_int;
    pub fn rk_stats_reset() -> c_int;
    pub fn rk_mem_stats(out: *mut RkMemStats) -> c_int;
    pub fn rk_trim_scratch_to(budget: u64) -> c_int;
    pub fn rk_clear_scratch() -> c_int;
    pub fn rk_trim_scratch() -> c_int;
    pub fn rk_pack(w: *const f32, n: i64, k: i64, id: *mut WeightId) -> c_int;
    pub fn rk_pack_f16(w: *const u16, n: i64, k: i64, id: *mut WeightId) -> c_int;
    pub fn rk_pack_seg(
        parts: *const *const f32, ns: *const i64, nparts: c_int, k: i64, id: *mut WeightId
    ) -> c_int;
    pub fn rk_pack_i8(w: *const f32, n: i64, k: i64, group: i64, id: *mut WeightId) -> c_int;
    pub fn rk_pack_i8_codes(
        codes: *const i8, scales: *const f32, n: i64, k: i64, group: i64, id: *mut WeightId
    ) -> c_int;
    pub fn rk_rewrite_i8(id: WeightId, codes: *const i8, scales: *const f32) -> c_int;
    pub fn rk_pack_q8_0(blocks: *const u8, n: i64, k: i64, id: *mut WeightId) -> c_int;
    pub fn rk_pack_q8_0_f32(w: *const f32, n: i64, k: i64, id: *mut WeightId) -> c_int;
    pub fn rk_pack_qat(
        codes: *const i8, w_scale: *const f32, n: i64, k: i64, in_scale: f32, out_scale: f32,
        id: *mut WeightId
    ) -> c_int;
    pub fn rk_weight_info(
        id: WeightId, kind: *mut c_int, n: *mut i64, k: *mut i64, group: *mut i64
    ) -> c_int;
    pub fn rk_matmul(id: WeightId, x: *const f32, m: i64, k: i64, y: *mut f32) -> c_int;
    pub fn rk_matmul_f16(id: WeightId, a: *const u16, m: i64, k: i64, c: *mut u16) -> c_int;
    pub fn rk_matmul_i8_gw(
        id: WeightId, a: *const i8, a_scale: *const f32, b_scale: *const f32, m: i64, k: i64,
        cf: *mut f32
    ) -> c_int;
    pub fn rk_matmul_i8(id: WeightId, a: *const i8, m: i64, k: i64, c: *mut i32) -> c_int;
    pub fn rk_matmul_f16_dev(
        id: WeightId, a: *const c_void, m: i64, k: i64, c: *mut c_void, stream: Stream
    ) -> c_int;
    pub fn rk_pack_f16_glu(gate: *const f32, up: *const f32, n: i64, k: i64, id: *mut WeightId) -> c_int;
    pub fn rk_matmul_f16_glu_dev(
        id: WeightId, a: *const c_void, m: i64, k: i64, glu: c_int, out: *mut c_void, out_f16: c_int,
        stream: Stream
    ) -> c_int;
    pub fn rk_quantize_rows_dev(
        x: *const f32, m: i64, k: i64, group: i64, q: *mut i8, scale: *mut f32, stream: Stream
    ) -> c_int;
    pub fn rk_matmul_w8a8_dev(
        id: WeightId, a: *const i8, a_scale: *const f32, a_group: i64, m: i64, k: i64, c: *mut f32,
        stream: Stream
    ) -> c_int;
    pub fn rk_matmul_w8a8_f16out_dev(
        id: WeightId, a: *const i8, a_scale: *const f32, a_group: i64, m: i64, k: i64,
        c: *mut c_void, stream: Stream
    ) -> c_int;
    pub fn rk_matmul_i8_raw_dev(
        id: WeightId, a: *const i8, m: i64, k: i64, c: *mut i32, stream: Stream
    ) -> c_int;
    pub fn rk_matmul_i8_partials_dev(
        id: WeightId, a: *const i8, m: i64, k: i64, p: *mut i32, stream: Stream
    ) -> c_int;
    pub fn rk_attention(
        q: *const f32, k: *const f32, v: *const f32, n_q: i64, n_kv: i64, n_head: c_int,
        n_kv_heads: c_int, head_dim: c_int, scale: f32, softcap: f32, mask_mode: c_int,
        window: i64, q0: i64, k0: i64, out: *mut f32
    ) -> c_int;
    pub fn rk_attention_dev(
        q: *const c_void, k: *const c_void, v: *const c_void, n_q: i64, n_kv: i64, n_head: c_int,
        n_kv_heads: c_int, head_dim: c_int, scale: f32, softcap: f32, mask_mode: c_int,
        window: i64, q0: i64, k0: i64, out: *mut c_void, stream: Stream
    ) -> c_int;
    pub fn rk_attention_dev_noalloc(
        q: *const c_void, k: *const c_void, v: *const c_void, n_q: i64, n_kv: i64, n_head: c_int,
        n_kv_heads: c_int, head_dim: c_int, scale: f32, softcap: f32, mask_mode: c_int,
        window: i64, q0: i64, k0: i64, out: *mut c_void, stream: Stream
    ) -> c_int;
    pub fn rk_attention_strided_dev(
        q: *const c_void, q_stride: i64, k: *const c_void, k_stride: i64, v: *const c_void,
        v_stride: i64, n_q: i64, n_kv: i64, n_head: c_int, n_kv_heads: c_int, head_dim: c_int,
        scale: f32, softcap: f32, mask_mode: c_int, window: i64, q0: i64, k0: i64,
        out: *mut c_void, out_stride: i64, stream: Stream
    ) -> c_int;
    pub fn rk_flash_attn_f16(
        n_q: i64, n_kv: i64, head_dim: c_int, dv: c_int, n_head: c_int, n_kv_heads: c_int,
        scale: f32, softcap: f32, mask_mode: c_int, window: i64, q0: i64, k0: i64, q: *const u16,
        k: *const u16, v: *const u16, out: *mut u16
    ) -> c_int;
    pub fn rk_flash_attn_f16_masked(
        n_q: i64, n_kv: i64, head_dim: c_int, dv: c_int, n_head: c_int, n_kv_heads: c_int,
        scale: f32, softcap: f32, mask: *const u16, q: *const u16, k: *const u16, v: *const u16,
        out: *mut u16
    ) -> c_int;
    pub fn rk_moe_route(
        logits: *const f32, s: i64, n_experts: c_int, top_k: c_int, norm_topk: c_int,
        ids: *mut u32, wts: *mut f32
    ) -> c_int;
    pub fn rk_pack_moe_q8_0(
        gate: *const u8, up: *const u8, down: *const u8, n_experts: c_int, hidden: i64, inter: i64,
        id: *mut WeightId
    ) -> c_int;
    pub fn rk_pack_moe_f32(
        gate: *const f32, up: *const f32, down: *const f32, n_experts: c_int, hidden: i64,
        inter: i64, id: *mut WeightId
    ) -> c_int;
    pub fn rk_moe_experts_dev(
        id: WeightId, x: *const f32, s: i64, top_k: c_int, ids: *const u32, wts: *const f32,
        y: *mut f32, stream: Stream
    ) -> c_int;
    pub fn rk_moe_experts_acc_dev(
        id: WeightId, x: *const f32, s: i64, top_k: c_int, ids: *const u32, wts: *const f32,
        y: *mut f32, stream: Stream
    ) -> c_int;
    pub fn rk_moe_plan_create(
        id: WeightId, s: i64, top_k: c_int, ids: *const u32, wts: *const f32,
        plan: *mut *mut c_void
    ) -> c_int;
    pub fn rk_moe_experts_planned_dev(
        id: WeightId, plan: *const c_void, x: *const f32, y: *mut f32, stream: Stream
    ) -> c_int;
    pub fn rk_moe_experts_planned_acc_dev(
        id: WeightId, plan: *const c_void, x: *const f32, y: *mut f32, stream: Stream
    ) -> c_int;
    pub fn rk_moe_plan_destroy(plan: *mut c_void) -> c_int;
    pub fn rk_moe_gate_up_dev(
        id: WeightId, plan: *const c_void, x: *const f32, act: *mut f32, stream: Stream
    ) -> c_int;
    pub fn rk_silu_mul_dev(
        a: *const c_void, b: *const c_void, out: *mut c_void, n: i64, dr#type: c_int,
        stream: Stream
    ) -> c_int;
    pub fn rk_gelu_mul_dev(
        a: *const c_void, b: *const c_void, out: *mut c_void, n: i64, dr#type: c_int,
        stream: Stream
    ) -> c_int;
    pub fn rk_silu_mul(a: *const f32, b: *const f32, out: *mut f32, n: i64) -> c_int;
    pub fn rk_gelu_mul(a: *const f32, b: *const f32, out: *mut f32, n: i64) -> c_int;
    pub fn rk_pack_q8_0_glu(
        gate_blocks: *const u8, up_blocks: *const u8, n: i64, k: i64, id: *mut WeightId
    ) -> c_int;
    pub fn rk_pack_q8_0_glu_f32(
        gate: *const f32, up: *const f32, n: i64, k: i64, id: *mut WeightId
    ) -> c_int;
    pub fn rk_matmul_w8a8_glu_dev(
        id: WeightId, a: *const i8, a_scale: *const f32, m: i64, k: i64, glu: c_int,
        out: *mut c_void, out_f16: c_int, stream: Stream
    ) -> c_int;
    pub fn rk_rms_norm_dev(
        x: *const c_void, w: *const c_void, w_dr#type: c_int, out: *mut c_void, rows: i64, d: i64,
        eps: f64, dr#type: c_int, stream: Stream
    ) -> c_int;
    pub fn rk_rms_norm_noscale_dev(
        x: *const c_void, out: *mut c_void, rows: i64, d: i64, eps: f64, dr#type: c_int,
        stream: Stream
    ) -> c_int;
    pub fn rk_rope_dev(
        x: *const c_void, cos: *const c_void, sin: *const c_void, cs_dr#type: c_int,
        out: *mut c_void, b: i64, s: i64, h: i64, d: i64, dr#type: c_int, stream: Stream
    ) -> c_int;
    pub fn rk_qk_norm_rope_dev(
        qkv: *mut c_void, s: i64, row_stride: i64, n_q_heads: c_int, n_kv_heads: c_int,
        head_dim: i64, q_norm_w: *const c_void, k_norm_w: *const c_void, eps: f64,
        cos: *const c_void, sin: *const c_void, cs_dr#type: c_int, dr#type: c_int, stream: Stream
    ) -> c_int;
    pub fn rk_attention_qkv_dev(
        qkv: *mut c_void, s: i64, row_stride: i64, n_head: c_int, n_kv_heads: c_int,
        head_dim: c_int, q_norm_w: *const c_void, k_norm_w: *const c_void, eps: f64,
        cos: *const c_void, sin: *const c_void, cs_dr#type: c_int, scale: f32, softcap: f32,
        mask_mode: c_int, window: i64, q0: i64, k0: i64, out: *mut c_void, out_stride: i64,
        stream: Stream
    ) -> c_int;
    pub fn rk_rms_norm_quantize_dev(
        x: *const c_void, w: *const c_void, w_dr#type: c_int, rows: i64, d: i64, eps: f64,
        dr#type: c_int, q: *mut i8, q_scale: *mut f32, stream: Stream
    ) -> c_int;
    pub fn rk_rms_norm(
        x: *const f32, w: *const f32, out: *mut f32, rows: i64, d: i64, eps: f64
    ) -> c_int;
    pub fn rk_rms_norm_noscale(x: *const f32, out: *mut f32, rows: i64, d: i64, eps: f64) -> c_int;
    pub fn rk_rope(
        x: *const f32, cos: *const f32, sin: *const f32, out: *mut f32, b: i64, s: i64, h: i64,
        d: i64
    ) -> c_int;
    pub fn rk_device_alloc(bytes: usize, ptr: *mut *mut c_void) -> c_int;
    pub fn rk_device_free(ptr: *mut c_void) -> c_int;
    pub fn rk_memcpy_htod(dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn rk_memcpy_dtoh(dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn rk_memcpy_dtod(
        dst: *mut c_void, src: *const c_void, bytes: usize, stream: Stream
    ) -> c_int;
    pub fn rk_cast_dev(
        x: *const c_void, x_dtype: c_int, y: *mut c_void, y_dtype: c_int, n: i64, stream: Stream
    ) -> c_int;
    pub fn rk_memset_dev(dst: *mut c_void, value: c_int, bytes: usize) -> c_int;
    pub fn rk_stream_get(stream: *mut Stream) -> c_int;
    pub fn rk_stream_create(stream: *mut Stream) -> c_int;
    pub fn rk_stream_destroy(stream: Stream) -> c_int;
    pub fn rk_stream_sync(stream: Stream) -> c_int;
    pub fn rk_event_create(event: *mut *mut c_void) -> c_int;
    pub fn rk_event_destroy(event: *mut c_void) -> c_int;
    pub fn rk_event_record(event: *mut c_void, stream: Stream) -> c_int;
    pub fn rk_event_elapsed_ms(start: *mut c_void, stop: *mut c_void, ms: *mut f32) -> c_int;
    pub fn rk_device_info(
        name: *mut c_char, name_len: usize, cus: *mut c_int, clock_khz: *mut c_int
    ) -> c_int;
}

/// A failed call: the op name and its status code, as `burn_rocket::Error`.
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub struct Error {
    pub op: &'static str,
    pub rc: i32,
}

impl Error {
    /// True when the caller may fall back to another path (`RK_E_TILING`).
    pub fn is_fallback(&self) -> bool {
        self.rc == RK_E_TILING
    }
}

impl std::fmt::Display for Error {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        let kind = match self.rc {
            RK_E_SHAPE => "unsupported shape",
            RK_E_TILING => "shape not tileable",
            RK_E_NOMEM => "allocation failed",
            RK_E_DEVICE => "device/driver failure",
            RK_E_UNSUPPORTED => "unsupported feature",
            RK_E_RANGE => "value out of range",
            RK_E_IO => "i/o failure",
            _ => "unknown error",
        };
        write!(f, "{} failed: {} (rc={})", self.op, kind, self.rc)
    }
}

impl std::error::Error for Error {}

/// The library's message for the last failure on this thread.
pub fn last_error() -> String {
    // SAFETY: rk_last_error returns a NUL-terminated string owned by the library
    // that stays valid until the next failing call on this thread.
    unsafe { CStr::from_ptr(rk_last_error()) }.to_string_lossy().into_owned()
}

fn check(rc: c_int, op: &'static str) -> Result<(), Error> {
    if rc == RK_OK { Ok(()) } else { Err(Error { op, rc }) }
}

/// `rk_init(device)`: the process-global engine (later calls are no-ops).
pub fn init(device: i32) -> Result<(), Error> {
    check(unsafe { rk_init(device) }, "rocket_init")
}

/// Resident fp16 weight from f32 `[n, k]` (`burn_rocket::pack`).
pub fn pack_f32(w: &[f32], n: usize, k: usize) -> Result<WeightId, Error> {
    assert_eq!(w.len(), n * k, "pack: weight must be [N, K]");
    let mut id = 0;
    check(unsafe { rk_pack(w.as_ptr(), n as i64, k as i64, &mut id) }, "rocket_weights_pack")?;
    Ok(id)
}

/// Segments `[n_i, k]` concatenated along N (`pack2` / `pack3`).
pub fn pack_seg(parts: &[(&[f32], usize)], k: usize) -> Result<WeightId, Error> {
    let ptrs: Vec<*const f32> = parts.iter().map(|(p, _)| p.as_ptr()).collect();
    let ns: Vec<i64> = parts.iter().map(|&(p, n)| {
        assert_eq!(p.len(), n * k, "pack_seg: every part must be [n_i, K]");
        n as i64
    }).collect();
    let mut id = 0;
    check(
        unsafe { rk_pack_seg(ptrs.as_ptr(), ns.as_ptr(), parts.len() as c_int, k as i64, &mut id) },
        "rocket_weights_pack_seg",
    )?;
    Ok(id)
}

/// Group-wise int8 weight quantized from f32 `[n, k]` (`burn_rocket::pack_i8`).
pub fn pack_i8(w: &[f32], n: usize, k: usize, group: usize) -> Result<WeightId, Error> {
    assert_eq!(w.len(), n * k, "pack_i8: weight must be [N, K]");
    let mut id = 0;
    check(
        unsafe { rk_pack_i8(w.as_ptr(), n as i64, k as i64, group as i64, &mut id) },
        "rocket_i8_weights_pack_gw",
    )?;
    Ok(id)
}

/// Per-channel QAT weight (`burn_rocket::pack_qat`).
pub fn pack_qat(
    codes: &[i8], w_scale: &[f32], n: usize, k: usize, in_scale: f32, out_scale: f32,
) -> Result<WeightId, Error> {
    assert_eq!(codes.len(), n * k, "pack_qat: codes must be [N, K]");
    assert_eq!(w_scale.len(), n, "pack_qat: one weight scale per output channel");
    let mut id = 0;
    check(
        unsafe {
            rk_pack_qat(codes.as_ptr(), w_scale.as_ptr(), n as i64, k as i64, in_scale, out_scale, &mut id)
        },
        "rocket_i8_weights_pack",
    )?;
    Ok(id)
}

/// (kind, n, k, group) of a resident weight.
pub fn weight_info(id: WeightId) -> Result<(i32, usize, usize, usize), Error> {
    let (mut kind, mut n, mut k, mut g) = (0, 0i64, 0i64, 0i64);
    check(unsafe { rk_weight_info(id, &mut kind, &mut n, &mut k, &mut g) }, "rocket_weight_info")?;
    Ok((kind, n as usize, k as usize, g as usize))
}

/// `y[m, n] = x[m, k] · Wᵀ` on host f32 buffers for any weight kind (`rocket_matmul`).
pub fn matmul(id: WeightId, x: &[f32], m: usize, k: usize, y: &mut [f32]) -> Result<(), Error> {
    assert_eq!(x.len(), m * k, "matmul: x must be [M, K]");
    // The library writes m·N values, N from the resident weight.
    let (_, n, wk, _) = weight_info(id)?;
    assert_eq!(wk, k, "matmul: activation K differs from the weight's K");
    assert_eq!(y.len(), m * n, "matmul: y must be [M, N]");
    check(unsafe { rk_matmul(id, x.as_ptr(), m as i64, k as i64, y.as_mut_ptr()) }, "rocket_matmul")
}

/// `C[m, n] = A[m, k] · Bᵀ` on host fp16 buffers (`RocketCtx::matmul_prepacked`).
pub fn matmul_f16(id: WeightId, a: &[u16], m: usize, k: usize, c: &mut [u16]) -> Result<(), Error> {
    let (kind, n, wk, _) = weight_info(id)?;
    assert_eq!(kind, RK_WEIGHT_F16, "matmul_f16: not an fp16 weight");
    assert_eq!(wk, k, "matmul_f16: activation K differs from the weight's K");
    assert!(a.len() == m * k && c.len() == m * n, "matmul_f16: A [M, K], C [M, N]");
    check(unsafe { rk_matmul_f16(id, a.as_ptr(), m as i64, k as i64, c.as_mut_ptr()) }, "rocket_matmul_fp16")
}

/// `cf[m, n] = Σ_g a_scale[m,g]·b_scale[n,g]·P_g` on host buffers (`I8Context::matmul_gw`);
/// `b_scale` None uses the scales packed with the weight.
pub fn matmul_i8_gw(
    id: WeightId, a: &[i8], a_scale: &[f32], b_scale: Option<&[f32]>, m: usize, k: usize, cf: &mut [f32],
) -> Result<(), Error> {
    let (kind, n, wk, group) = weight_info(id)?;
    assert!(kind == RK_WEIGHT_I8 && group > 0, "matmul_i8_gw: not a group-wise int8 weight");
    assert_eq!(wk, k, "matmul_i8_gw: activation K differs from the weight's K");
    let ng = k / group;
    assert!(a.len() == m * k && a_scale.len() == m * ng && cf.len() == m * n, "matmul_i8_gw: buffers");
    if let Some(b) = b_scale {
        assert_eq!(b.len(), n * ng, "matmul_i8_gw: b_scale must be [N, K/group]");
    }
    let bp = b_scale.map_or(std::ptr::null(), |b| b.as_ptr());
    check(
        unsafe { rk_matmul_i8_gw(id, a.as_ptr(), a_scale.as_ptr(), bp, m as i64, k as i64, cf.as_mut_ptr()) },
        "rocket_matmul_int8_prepacked_gw",
    )
}

/// Raw int32 `c[m, n] = Σ_k a[m,k]·w[n,k]` on host buffers (`I8Context::matmul`).
pub fn matmul_i8(id: WeightId, a: &[i8], m: usize, k: usize, c: &mut [i32]) -> Result<(), Error> {
    let (kind, n, wk, _) = weight_info(id)?;
    assert!(kind == RK_WEIGHT_I8 || kind == RK_WEIGHT_QAT, "matmul_i8: not an int8 weight");
    assert_eq!(wk, k, "matmul_i8: activation K differs from the weight's K");
    assert!(a.len() == m * k && c.len() == m * n, "matmul_i8: A [M, K], C [M, N]");
    check(unsafe { rk_matmul_i8(id, a.as_ptr(), m as i64, k as i64, c.as_mut_ptr()) }, "rocket_matmul_int8_prepacked")
}

/// Resident fp16 weight from fp16 bits `[n, k]` (`RocketCtx::pack_weight`).
pub fn pack_f16(w: &[u16], n: usize, k: usize) -> Result<WeightId, Error> {
    assert_eq!(w.len(), n * k, "pack_f16: weight must be [N, K]");
    let mut id = 0;
    check(unsafe { rk_pack_f16(w.as_ptr(), n as i64, k as i64, &mut id) }, "rocket_weights_pack")?;
    Ok(id)
}

/// Group-wise int8 codes `[n, k]`, with scales `[n, k/group]` or without
/// (`I8Context::pack_weight_gw` keeps the codes alone).
pub fn pack_i8_codes(codes: &[i8], scales: Option<&[f32]>, n: usize, k: usize, group: usize) -> Result<WeightId, Error> {
    assert_eq!(codes.len(), n * k, "pack_i8_codes: codes must be [N, K]");
    assert!(group > 0 && group % 32 == 0 && k % group == 0, "pack_i8_codes: group");
    if let Some(s) = scales {
        assert_eq!(s.len(), n * (k / group), "pack_i8_codes: scales must be [N, K/group]");
    }
    let sp = scales.map_or(std::ptr::null(), |s| s.as_ptr());
    let mut id = 0;
    check(
        unsafe { rk_pack_i8_codes(codes.as_ptr(), sp, n as i64, k as i64, group as i64, &mut id) },
        "rocket_i8_weights_pack_gw",
    )?;
    Ok(id)
}

/// New codes (and scales, or keep the resident ones) for a resident int8 weight.
pub fn rewrite_i8(id: WeightId, codes: &[i8], scales: Option<&[f32]>) -> Result<(), Error> {
    let (_, n, k, group) = weight_info(id)?;
    assert_eq!(codes.len(), n * k, "rewrite_i8: codes must be [N, K]");
    if let Some(s) = scales {
        assert_eq!(s.len(), n * (k / group), "rewrite_i8: scales must be [N, K/group]");
    }
    let sp = scales.map_or(std::ptr::null(), |s| s.as_ptr());
    check(unsafe { rk_rewrite_i8(id, codes.as_ptr(), sp) }, "rocket_i8_rewrite_gw")
}

/// Head-major fp16 attention with an optional additive 0 / -inf mask
/// (`RocketFaCtx::flash_attn`): q `[H][n_q][head_dim]`, k `[KV][n_kv][head_dim]`,
/// v `[KV][dv][n_kv]`, out `[H][n_q][dv]`, mask `[n_q][n_kv]`.
#[allow(clippy::too_many_arguments)]
pub fn flash_attn_f16(
    n_q: usize, n_kv: usize, head_dim: usize, dv: usize, n_head: usize, n_kv_heads: usize, scale: f32,
    softcap: f32, q: &[u16], k: &[u16], v: &[u16], mask: Option<&[u16]>, out: &mut [u16],
) -> Result<(), Error> {
    assert_eq!(q.len(), n_head * n_q * head_dim, "flash_attn: q must be [H][n_q][head_dim]");
    assert_eq!(k.len(), n_kv_heads * n_kv * head_dim, "flash_attn: k must be [KV][n_kv][head_dim]");
    assert_eq!(v.len(), n_kv_heads * dv * n_kv, "flash_attn: v must be [KV][dv][n_kv]");
    assert_eq!(out.len(), n_head * n_q * dv, "flash_attn: out must be [H][n_q][dv]");
    if let Some(m) = mask {
        assert_eq!(m.len(), n_q * n_kv, "flash_attn: mask must be [n_q][n_kv]");
    }
    let mp = mask.map_or(std::ptr::null(), |m| m.as_ptr());
    check(
        unsafe {
            rk_flash_attn_f16_masked(
                n_q as i64, n_kv as i64, head_dim as c_int, dv as c_int, n_head as c_int, n_kv_heads as c_int,
                scale, softcap, mp, q.as_ptr(), k.as_ptr(), v.as_ptr(), out.as_mut_ptr(),
            )
        },
        "rocket_flash_attn_fp16_ctx",
    )
}

/// The mask of one attention call: mode, window and the block offsets.
#[derive(Debug, Clone, Copy)]
pub struct Mask {
    pub mode: c_int,
    pub window: i64,
    pub q0: i64,
    pub k0: i64,
}

/// Masked GQA attention on token-major host f32 buffers (`rocket_attention*`).
#[allow(clippy::too_many_arguments)]
pub fn attention(
    q: &[f32], k: &[f32], v: &[f32], n_q: usize, n_kv: usize, n_head: usize, n_kv_heads: usize,
    head_dim: usize, scale: f32, softcap: f32, mask: Mask, out: &mut [f32],
) -> Result<(), Error> {
    assert_eq!(q.len(), n_q * n_head * head_dim, "attention: q must be [S, H*D]");
    assert_eq!(k.len(), n_kv * n_kv_heads * head_dim, "attention: k must be [S_k, KV*D]");
    assert_eq!(v.len(), k.len(), "attention: v must be [S_k, KV*D]");
    assert_eq!(out.len(), q.len(), "attention: out must be [S, H*D]");
    check(
        unsafe {
            rk_attention(
                q.as_ptr(), k.as_ptr(), v.as_ptr(), n_q as i64, n_kv as i64, n_head as c_int,
                n_kv_heads as c_int, head_dim as c_int, scale, softcap, mask.mode, mask.window,
                mask.q0, mask.k0, out.as_mut_ptr(),
            )
        },
        "rocket_flash_attn_fp16_ctx",
    )
}

/// `silu(a)·b` / `gelu_tanh(a)·b` on host f32 buffers.
pub fn silu_mul(a: &[f32], b: &[f32], out: &mut [f32]) -> Result<(), Error> {
    assert!(a.len() == b.len() && b.len() == out.len(), "silu_mul: equal lengths");
    check(unsafe { rk_silu_mul(a.as_ptr(), b.as_ptr(), out.as_mut_ptr(), a.len() as i64) }, "rocket_silu_mul")
}
pub fn gelu_mul(a: &[f32], b: &[f32], out: &mut [f32]) -> Result<(), Error> {
    assert!(a.len() == b.len() && b.len() == out.len(), "gelu_mul: equal lengths");
    check(unsafe { rk_gelu_mul(a.as_ptr(), b.as_ptr(), out.as_mut_ptr(), a.len() as i64) }, "rocket_gelu_mul")
}

/// RMSNorm over rows of `d` values on host f32 buffers (`w` None: scale-free).
pub fn rms_norm(x: &[f32], w: Option<&[f32]>, d: usize, eps: f64, out: &mut [f32]) -> Result<(), Error> {
    assert!(d > 0 && x.len() % d == 0 && out.len() == x.len(), "rms_norm: rows of d values");
    let rows = (x.len() / d) as i64;
    match w {
        Some(w) => {
            assert_eq!(w.len(), d, "rms_norm: the weight has the last dim's size");
            check(
                unsafe { rk_rms_norm(x.as_ptr(), w.as_ptr(), out.as_mut_ptr(), rows, d as i64, eps) },
                "rocket_rms_norm",
            )
        }
        None => check(
            unsafe { rk_rms_norm_noscale(x.as_ptr(), out.as_mut_ptr(), rows, d as i64, eps) },
            "rocket_rms_norm_noscale",
        ),
    }
}

/// Rotate-half RoPE of `x [b, s, h, d]` with `cos`/`sin` `[s, d/2]` on host f32 buffers.
#[allow(clippy::too_many_arguments)]
pub fn rope(
    x: &[f32], cos: &[f32], sin: &[f32], b: usize, s: usize, h: usize, d: usize, out: &mut [f32],
) -> Result<(), Error> {
    assert_eq!(x.len(), b * s * h * d, "rope: x must be [B, S, H, D]");
    assert_eq!(out.len(), x.len(), "rope: out must be [B, S, H, D]");
    assert!(cos.len() == s * d / 2 && sin.len() == s * d / 2, "rope: tables must be [S, D/2]");
    check(
        unsafe {
            rk_rope(x.as_ptr(), cos.as_ptr(), sin.as_ptr(), out.as_mut_ptr(), b as i64, s as i64,
                    h as i64, d as i64)
        },
        "rocket_rope",
    )
}

pub fn stats() -> Result<RkStats, Error> {
    let mut s = RkStats::default();
    check(unsafe { rk_stats(&mut s) }, "stats")?;
    Ok(s)
}
pub fn stats_reset() -> Result<(), Error> {
    check(unsafe { rk_stats_reset() }, "stats_reset")
}
pub fn mem_stats() -> Result<RkMemStats, Error> {
    let mut s = RkMemStats::default();
    check(unsafe { rk_mem_stats(&mut s) }, "mem_stats")?;
    Ok(s)
}
pub fn trim_scratch_to(budget: u64) -> Result<(), Error> {
    check(unsafe { rk_trim_scratch_to(budget) }, "trim_scratch_to")
}
pub fn clear_scratch() -> Result<(), Error> {
    check(unsafe { rk_clear_scratch() }, "clear_scratch")
}
pub fn trim_scratch() -> Result<(), Error> {
    check(unsafe { rk_trim_scratch() }, "trim_scratch")
}

pub mod ctx;
pub mod npu;
pub use ctx::{RocketCtx, RocketFaCtx, RocketWeight};
