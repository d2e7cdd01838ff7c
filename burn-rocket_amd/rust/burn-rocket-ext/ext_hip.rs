//! `impl RocketOps for Flex` on the MI355X library, through `rocket-hip-sys`.
//!
//! A drop-in for the RK3588 bodies of `crates/burn-rocket/src/ext.rs`: the
//! `Flex` impl (ext.rs:586-756), `init` (ext.rs:561-580) and the op bodies it
//! calls (pack_one / pack_many ext.rs:829-934, pack_i8_one ext.rs:939-1012,
//! matmul_impl ext.rs:1208-1232, attention_impl ext.rs:1669-1858, the glue
//! ops ext.rs:1057-1152). The trait (ext.rs:57-164), `WeightId`, the helper API
//! (ext.rs:1864-2137) and the error types keep their signatures, so model code
//! and `--device` placement are unchanged. Placed in `crates/burn-rocket/src/`
//! as a module of `ext.rs` (`mod ext_hip;` with the RK3588 impl removed) and
//! with `rocket-hip-sys` as a dependency.
//!
//! Tensors arrive as owned host primitives (as today, ext.rs:759-779); their
//! f32 values cross the C ABI and the library converts and quantizes on the GPU.
//! A failed call aborts the op with `panic_any(OpFailure { .. })`, as
//! `op_failure` does (ext.rs:344-352). Weights in bf16 are packed as fp16
//! (the bf16 streaming context of the reference is not part of this library).
//!
//! Beside the trait, the free functions the app calls whose reference bodies
//! reach the RK3588 engine are replaced too: `pack_qat`, `stats`,
//! `stats_reset`, `mem_stats`, `trim_scratch`, `trim_scratch_to` and
//! `clear_scratch`. The driver types Clef holds directly (`RocketCtx`,
//! `RocketFaCtx`, `npu::matmul::I8Context`) come from rocket-hip-sys
//! (`ctx.rs`, `npu.rs`), re-exported by lib.rs in place of rocket-npu's.
//!
//! Not compiled in the repository that holds it (no Rust toolchain there);
//! tests/test_rust_binding.py checks that every item it takes from
//! rocket-hip-sys exists there, and that the crate's FFI declarations match
//! include/burn_rocket_amd.h.

use burn::backend::tensor::FloatTensor;
use burn::backend::{Flex, TensorMetadata};
use burn::tensor::{DType, TensorData};
use half::{bf16, f16};
use rocket_hip_sys as hip;

use super::RocketOps;
use crate::{Error, OpFailure};

type FlexTensor = FloatTensor<Flex>;

/// Abort the op with the structured payload the serving layer maps to a response.
fn op_failure(e: hip::Error, m: usize, k: usize, n: usize) -> ! {
    eprintln!("burn-rocket: {e}: {} (m={m} k={k} n={n})", hip::last_error());
    std::panic::panic_any(OpFailure { error: Error { op: e.op, rc: e.rc }, m, k, n })
}

/// `burn_rocket::init`: the engine on HIP device 0 (the worker count of the
/// NPU driver has no counterpart; the GPU schedules its own work).
pub fn init(_threads: usize) -> Result<(), Error> {
    hip::init(0).map_err(|e| Error { op: e.op, rc: e.rc })
}

/// Shape, f32 values and dtype of an f32 / f16 / bf16 tensor.
fn read_f32(t: FlexTensor, what: &str) -> (Vec<usize>, Vec<f32>, DType) {
    let dims: Vec<usize> = t.shape().into();
    let dtype = t.dtype();
    let values = match dtype {
        DType::F32 => t.into_data().try_to_vec::<f32>().unwrap_or_else(|e| panic!("{what}: {e}")),
        DType::F16 => t
            .into_data()
            .try_to_vec::<f16>()
            .unwrap_or_else(|e| panic!("{what}: {e}"))
            .into_iter()
            .map(f16::to_f32)
            .collect(),
        DType::BF16 => t
            .into_data()
            .try_to_vec::<bf16>()
            .unwrap_or_else(|e| panic!("{what}: {e}"))
            .into_iter()
            .map(bf16::to_f32)
            .collect(),
        other => panic!("{what}: unsupported float dtype {other:?} (f32/f16/bf16)"),
    };
    (dims, values, dtype)
}

/// A float tensor of the requested dtype from f32 values (RNE for f16 / bf16).
fn floats_tensor(values: Vec<f32>, dims: Vec<usize>, dtype: DType) -> FlexTensor {
    match dtype {
        DType::F32 => FlexTensor::from_data(TensorData::new(values, dims)),
        DType::F16 => {
            let v: Vec<f16> = values.into_iter().map(f16::from_f32).collect();
            FlexTensor::from_data(TensorData::new(v, dims))
        }
        DType::BF16 => {
            let v: Vec<bf16> = values.into_iter().map(bf16::from_f32).collect();
            FlexTensor::from_data(TensorData::new(v, dims))
        }
        other => panic!("unsupported output dtype {other:?} (f32/f16/bf16)"),
    }
}

fn weight_nk(t: FlexTensor, what: &str) -> (usize, usize, Vec<f32>) {
    let (dims, w, _) = read_f32(t, what);
    assert_eq!(dims.len(), 2, "{what}: weights are [N, K]");
    (dims[0], dims[1], w)
}

fn pack_many(parts: Vec<FlexTensor>) -> u64 {
    let parts: Vec<(usize, usize, Vec<f32>)> = parts.into_iter().map(|t| weight_nk(t, "fused weight")).collect();
    let k = parts[0].1;
    assert!(parts.iter().all(|p| p.1 == k), "fused weight: all parts must share K");
    let segs: Vec<(&[f32], usize)> = parts.iter().map(|(n, _, w)| (w.as_slice(), *n)).collect();
    let n: usize = parts.iter().map(|p| p.0).sum();
    hip::pack_seg(&segs, k).unwrap_or_else(|e| op_failure(e, 0, k, n))
}

/// The library's mask encoding of one reference mask mode (ext.rs:1643-1666).
fn mask(mode: i32, window: i64, q0: i64, k0: i64) -> hip::Mask {
    hip::Mask { mode, window, q0: q0.max(0), k0: k0.max(0) }
}

#[allow(clippy::too_many_arguments)]
fn attention_impl(
    q: FlexTensor, k: FlexTensor, v: FlexTensor, n_head: usize, n_kv: usize, head_dim: usize,
    scale: f64, softcap: Option<f32>, m: hip::Mask,
) -> FlexTensor {
    let (q_dims, qv, out_dtype) = read_f32(q, "attention q");
    let (k_dims, kv, _) = read_f32(k, "attention k");
    let (v_dims, vv, _) = read_f32(v, "attention v");
    assert_eq!(q_dims.len(), 3, "attention input must be [1, S, H*D]");
    assert_eq!(q_dims[0], 1, "the attention path supports batch size 1");
    assert_eq!(q_dims[2], n_head * head_dim, "q width must be n_head * head_dim");
    let (n, n_k) = (q_dims[1], k_dims[1]);
    assert_eq!(k_dims, vec![1, n_k, n_kv * head_dim], "attention: k must be [1, S, KV*D]");
    assert_eq!(v_dims, k_dims, "attention: v must be [1, S, KV*D]");
    let mut out = vec![0f32; qv.len()];
    hip::attention(&qv, &kv, &vv, n, n_k, n_head, n_kv, head_dim, scale as f32, softcap.unwrap_or(0.0), m, &mut out)
        .unwrap_or_else(|e| op_failure(e, n, n_k, head_dim));
    floats_tensor(out, q_dims, out_dtype)
}

impl RocketOps for Flex {
    fn rocket_pack(t: FloatTensor<Self>) -> u64 {
        let (n, k, w) = weight_nk(t, "weight");
        hip::pack_f32(&w, n, k).unwrap_or_else(|e| op_failure(e, 0, k, n))
    }

    fn rocket_pack2(a: FloatTensor<Self>, b: FloatTensor<Self>) -> u64 {
        pack_many(vec![a, b])
    }

    fn rocket_pack3(a: FloatTensor<Self>, b: FloatTensor<Self>, c: FloatTensor<Self>) -> u64 {
        pack_many(vec![a, b, c])
    }

    fn rocket_pack_i8(t: FloatTensor<Self>, group: usize) -> u64 {
        let (n, k, w) = weight_nk(t, "int8 weight");
        assert!(group > 0 && group % 32 == 0 && k % group == 0, "int8 group {group} must be a multiple of 32 dividing K={k}");
        hip::pack_i8(&w, n, k, group).unwrap_or_else(|e| op_failure(e, 0, k, n))
    }

    fn rocket_gelu_mul(a: FloatTensor<Self>, b: FloatTensor<Self>) -> FloatTensor<Self> {
        let (dims, av, dtype) = read_f32(a, "gelu_mul a");
        let (b_dims, bv, _) = read_f32(b, "gelu_mul b");
        assert_eq!(dims, b_dims, "gelu_mul: inputs must share a shape");
        let mut out = vec![0f32; av.len()];
        hip::gelu_mul(&av, &bv, &mut out).unwrap_or_else(|e| op_failure(e, av.len(), 0, 0));
        floats_tensor(out, dims, dtype)
    }

    fn rocket_silu_mul(a: FloatTensor<Self>, b: FloatTensor<Self>) -> FloatTensor<Self> {
        let (dims, av, dtype) = read_f32(a, "silu_mul a");
        let (b_dims, bv, _) = read_f32(b, "silu_mul b");
        assert_eq!(dims, b_dims, "silu_mul: inputs must share a shape");
        let mut out = vec![0f32; av.len()];
        hip::silu_mul(&av, &bv, &mut out).unwrap_or_else(|e| op_failure(e, av.len(), 0, 0));
        floats_tensor(out, dims, dtype)
    }

    fn rocket_rms_norm(x: FloatTensor<Self>, w: FloatTensor<Self>, eps: f64) -> FloatTensor<Self> {
        let (dims, xv, dtype) = read_f32(x, "rms_norm x");
        let (_, wv, _) = read_f32(w, "rms_norm w");
        let d = *dims.last().expect("rms_norm needs at least one dim");
        let mut out = vec![0f32; xv.len()];
        hip::rms_norm(&xv, Some(&wv), d, eps, &mut out).unwrap_or_else(|e| op_failure(e, xv.len() / d, d, 0));
        floats_tensor(out, dims, dtype)
    }

    fn rocket_rms_norm_noscale(x: FloatTensor<Self>, eps: f64) -> FloatTensor<Self> {
        let (dims, xv, dtype) = read_f32(x, "rms_norm_noscale x");
        let d = *dims.last().expect("rms_norm needs at least one dim");
        let mut out = vec![0f32; xv.len()];
        hip::rms_norm(&xv, None, d, eps, &mut out).unwrap_or_else(|e| op_failure(e, xv.len() / d, d, 0));
        floats_tensor(out, dims, dtype)
    }

    fn rocket_rope(x: FloatTensor<Self>, cos: FloatTensor<Self>, sin: FloatTensor<Self>) -> FloatTensor<Self> {
        let (dims, xv, dtype) = read_f32(x, "rope x");
        let (_, cv, _) = read_f32(cos, "rope cos");
        let (_, sv, _) = read_f32(sin, "rope sin");
        assert_eq!(dims.len(), 4, "rope: x must be [B, S, H, D]");
        let (b, s, h, d) = (dims[0], dims[1], dims[2], dims[3]);
        let mut out = vec![0f32; xv.len()];
        hip::rope(&xv, &cv, &sv, b, s, h, d, &mut out).unwrap_or_else(|e| op_failure(e, b * s * h, d, 0));
        floats_tensor(out, dims, dtype)
    }

    fn rocket_matmul(x: FloatTensor<Self>, id: u64) -> FloatTensor<Self> {
        let (mut dims, xv, out_dtype) = read_f32(x, "matmul activations");
        assert!(dims.len() >= 2, "matmul needs at least [M, K]");
        let k = dims[dims.len() - 1];
        let m: usize = dims[..dims.len() - 1].iter().product();
        let (_, n, wk, _) = hip::weight_info(id).unwrap_or_else(|e| op_failure(e, m, k, 0));
        assert_eq!(wk, k, "matmul: activation K mismatch for weight id {id}");
        let mut y = vec![0f32; m * n];
        hip::matmul(id, &xv, m, k, &mut y).unwrap_or_else(|e| op_failure(e, m, k, n));
        *dims.last_mut().unwrap() = n;
        floats_tensor(y, dims, out_dtype)
    }

    fn rocket_attention(
        q: FloatTensor<Self>, k: FloatTensor<Self>, v: FloatTensor<Self>, n_head: usize,
        n_kv_heads: usize, head_dim: usize, scale: f64, softcap: Option<f32>, is_causal: bool,
    ) -> FloatTensor<Self> {
        let mode = if is_causal { hip::RK_MASK_CAUSAL } else { hip::RK_MASK_NONE };
        attention_impl(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, mask(mode, -1, 0, 0))
    }

    fn rocket_attention_window(
        q: FloatTensor<Self>, k: FloatTensor<Self>, v: FloatTensor<Self>, n_head: usize,
        n_kv_heads: usize, head_dim: usize, scale: f64, softcap: Option<f32>, window: i64,
    ) -> FloatTensor<Self> {
        // window < 0: no mask (the library maps the window mode to NONE)
        attention_impl(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, mask(hip::RK_MASK_WINDOW, window, 0, 0))
    }

    fn rocket_attention_causal_window(
        q: FloatTensor<Self>, k: FloatTensor<Self>, v: FloatTensor<Self>, n_head: usize,
        n_kv_heads: usize, head_dim: usize, scale: f64, softcap: Option<f32>, window: i64,
    ) -> FloatTensor<Self> {
        // window < 0: plain causal
        let m = mask(hip::RK_MASK_CAUSAL_WINDOW, window, 0, 0);
        attention_impl(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, m)
    }

    fn rocket_attention_window_block(
        q: FloatTensor<Self>, k: FloatTensor<Self>, v: FloatTensor<Self>, n_head: usize,
        n_kv_heads: usize, head_dim: usize, scale: f64, softcap: Option<f32>, window: i64,
        q_start: i64, kv_start: i64,
    ) -> FloatTensor<Self> {
        let m = mask(hip::RK_MASK_WINDOW, window, q_start, kv_start);
        attention_impl(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, m)
    }

    fn rocket_attention_causal_block(
        q: FloatTensor<Self>, k: FloatTensor<Self>, v: FloatTensor<Self>, n_head: usize,
        n_kv_heads: usize, head_dim: usize, scale: f64, softcap: Option<f32>, window: i64,
        q_start: i64, kv_start: i64,
    ) -> FloatTensor<Self> {
        let mode = if window >= 0 { hip::RK_MASK_CAUSAL_WINDOW } else { hip::RK_MASK_CAUSAL };
        attention_impl(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, mask(mode, window, q_start, kv_start))
    }
}

/// `burn_rocket::stats()` (ext.rs:176-193): conversion and device seconds of
/// the host-buffer ops and the matmul / attention / MoE call count.
pub fn stats() -> crate::Stats {
    let s = hip::stats().unwrap_or_default();
    crate::Stats { convert_s: s.convert_s, npu_s: s.device_s, calls: s.calls }
}

/// `burn_rocket::stats_reset()` (ext.rs:196-200).
pub fn stats_reset() {
    let _ = hip::stats_reset();
}

/// `burn_rocket::trim_scratch_to` / `clear_scratch` (ext.rs:256-308).
pub fn trim_scratch_to(budget: usize) {
    let _ = hip::trim_scratch_to(budget as u64);
}
pub fn clear_scratch() {
    let _ = hip::clear_scratch();
}

/// `burn_rocket::trim_scratch` (ext.rs:254-265): scratch no call used since the
/// previous trim goes; the just-used set stays (src/util/mem.rs:99-101 calls it
/// after each served request).
pub fn trim_scratch() {
    let _ = hip::trim_scratch();
}

/// `burn_rocket::mem_stats` (ext.rs:206-252): `None` before `init`, as the
/// reference. The device scratch splits into the attention buffers
/// (`attention_bo_bytes`) and the rest (`matmul_bo_bytes`); the page-locked
/// staging of the host-buffer ops is `matmul_host_bytes`. The scratch is one
/// buffer per use grown to its largest call, not a per-shape cache, so
/// `slots` and `attn_workers` stay empty.
pub fn mem_stats() -> Option<crate::MemStats> {
    let s = hip::mem_stats().ok()?;
    Some(crate::MemStats {
        weights_bytes: s.weights_bytes as usize,
        matmul_bo_bytes: (s.scratch_bytes - s.attention_bytes) as usize,
        matmul_host_bytes: s.host_bytes as usize,
        attention_bo_bytes: s.attention_bytes as usize,
        attention_host_bytes: 0,
        slots: Vec::new(),
        attn_workers: Vec::new(),
    })
}

/// `burn_rocket::pack_qat` (ext.rs:1375-1425): one pre-quantized per-channel
/// int8 weight of a QAT checkpoint, codes `[N, K]`, `w_scale [N]`, the static
/// activation scale (0 = per-row dynamic) and the output grid (0 = none). The
/// Gemma 4 loader packs its QAT linears through it
/// (src/gemma/gemma4/loader.rs:1149, 1283); `matmul` on the returned id runs
/// the QAT path (quantizer, exact int32 product, epilogue) on the GPU.
pub fn pack_qat(codes: &[i8], w_scale: Vec<f32>, n: usize, k: usize, in_scale: f32, out_scale: f32) -> super::WeightId {
    assert_eq!(codes.len(), n * k, "QAT codes must be [N, K]");
    assert_eq!(w_scale.len(), n, "one weight scale per output channel");
    assert!(in_scale >= 0.0, "QAT input scale must not be negative");
    assert_eq!(k % 32, 0, "the int8 path needs K % 32 == 0 (K={k})");
    assert_eq!(n % 32, 0, "the int8 path needs N % 32 == 0 (N={n})");
    let id = hip::pack_qat(codes, &w_scale, n, k, in_scale, out_scale).unwrap_or_else(|e| op_failure(e, 0, k, n));
    super::WeightId(id)
}
