//! `RocketCtx`, `RocketWeight` and `RocketFaCtx` (crates/burn-rocket/src/lib.rs:203-330)
//! over the MI355X library: the wrappers Clef's vision tower holds directly
//! (src/clef/vision/npu.rs:27, 89-248). `crates/burn-rocket` re-exports them
//! (`pub use rocket_hip_sys::{RocketCtx, RocketFaCtx, RocketWeight};`) in place of
//! its NPU-backed definitions, with the same methods and results.
//!
//! Buffers stay host fp16 slices as in the reference; the library stages them
//! through page-locked memory. Shape mismatches return `Err` with the shape
//! status, as the driver does (`Error::shape`, error.rs:95-97).

use half::f16;

use crate::{Error, WeightId, RK_E_SHAPE};

fn shape(op: &'static str) -> Error {
    Error { op, rc: RK_E_SHAPE }
}

fn bits(v: &[f16]) -> &[u16] {
    // SAFETY: f16 is a transparent wrapper of u16 (half 2.x), same size and alignment.
    unsafe { std::slice::from_raw_parts(v.as_ptr().cast::<u16>(), v.len()) }
}

fn bits_mut(v: &mut [f16]) -> &mut [u16] {
    // SAFETY: as in `bits`; the borrow is exclusive for the returned lifetime.
    unsafe { std::slice::from_raw_parts_mut(v.as_mut_ptr().cast::<u16>(), v.len()) }
}

/// Live scratch of a context: device bytes and page-locked host bytes
/// (`bo_bytes` / `host_bytes` of the driver's `MemStats`).
#[derive(Debug, Clone, Copy, Default)]
pub struct MemStats {
    pub bo_bytes: usize,
    pub host_bytes: usize,
}

/// A resident fp16 weight `[N, K]` (`RocketWeight`, lib.rs:268-270).
pub struct RocketWeight {
    id: WeightId,
    k: usize,
    n: usize,
}

impl RocketWeight {
    pub fn bytes(&self) -> usize {
        self.n * self.k * 2
    }

    pub fn id(&self) -> WeightId {
        self.id
    }
}

/// `RocketCtx` (lib.rs:203-266): resident fp16 weights and their GEMM.
pub struct RocketCtx {
    _engine: (),
}

impl RocketCtx {
    /// The engine on device 0; the NPU worker count has no counterpart.
    pub fn new(_nthreads: usize) -> Result<Self, Error> {
        crate::init(0)?;
        Ok(Self { _engine: () })
    }

    /// Pack `B [N, K]` (fp16, row-major) once; serves any M.
    pub fn pack_weight(&mut self, _m: usize, k: usize, n: usize, b: &[f16]) -> Result<RocketWeight, Error> {
        if b.len() != n * k {
            return Err(shape("rocket_weights_pack"));
        }
        Ok(RocketWeight { id: crate::pack_f16(bits(b), n, k)?, k, n })
    }

    /// Several weights sharing one input, concatenated along N.
    pub fn pack_weight_seg(&mut self, m: usize, k: usize, parts: &[&[f16]]) -> Result<RocketWeight, Error> {
        if parts.is_empty() || parts.iter().any(|p| p.is_empty() || p.len() % k != 0) {
            return Err(shape("rocket_weights_pack_seg"));
        }
        let all: Vec<f16> = parts.iter().flat_map(|p| p.iter().copied()).collect();
        self.pack_weight(m, k, all.len() / k, &all)
    }

    /// `C[M, N] = A[M, K]·B[N, K]ᵀ`, fp16 in and out, f32 accumulation; any M.
    pub fn matmul_prepacked(
        &mut self, m: usize, k: usize, n: usize, a: &[f16], c: &mut [f16], w: &RocketWeight,
    ) -> Result<(), Error> {
        if k != w.k || n != w.n || a.len() != m * k || c.len() != m * n {
            return Err(shape("rocket_matmul_fp16"));
        }
        crate::matmul_f16(w.id, bits(a), m, k, bits_mut(c))
    }

    /// Scratch not used since the previous trim goes; the just-used set stays.
    pub fn trim_scratch(&mut self) {
        let _ = crate::trim_scratch();
    }

    /// Evict scratch, largest first, until at most `budget` bytes remain.
    pub fn trim_to_budget(&mut self, budget: usize) {
        let _ = crate::trim_scratch_to(budget as u64);
    }

    pub fn scratch_bytes(&self) -> usize {
        let m = self.mem_stats();
        m.bo_bytes + m.host_bytes
    }

    pub fn clear_scratch(&mut self) {
        let _ = crate::clear_scratch();
    }

    pub fn mem_stats(&self) -> MemStats {
        crate::mem_stats()
            .map(|s| MemStats {
                bo_bytes: (s.scratch_bytes - s.attention_bytes) as usize,
                host_bytes: s.host_bytes as usize,
            })
            .unwrap_or_default()
    }
}

/// `RocketFaCtx` (lib.rs:282-330): head-major masked GQA attention.
pub struct RocketFaCtx {
    _engine: (),
}

impl RocketFaCtx {
    pub fn new(_nthreads: usize) -> Result<Self, Error> {
        crate::init(0)?;
        Ok(Self { _engine: () })
    }

    /// q `[H][T][head_dim]`, k `[KV][Nk][head_dim]`, v `[KV][dv][Nk]`, out
    /// `[H][T][dv]`; `mask` an additive `[T][Nk]` of 0 / -inf as the
    /// reference's builders make it (masks.rs), or None. Other masks return
    /// the unsupported status.
    #[allow(clippy::too_many_arguments)]
    pub fn flash_attn(
        &mut self, n_tokens: usize, n_kv: usize, head_dim: usize, dv: usize, n_head: usize, n_kv_heads: usize,
        scale: f32, softcap: f32, q: &[f16], k: &[f16], v: &[f16], mask: Option<&[f16]>, out: &mut [f16],
    ) -> Result<(), Error> {
        if q.len() != n_head * n_tokens * head_dim
            || k.len() != n_kv_heads * n_kv * head_dim
            || v.len() != n_kv_heads * dv * n_kv
            || out.len() != n_head * n_tokens * dv
            || mask.is_some_and(|m| m.len() != n_tokens * n_kv)
        {
            return Err(shape("rocket_flash_attn_fp16_ctx"));
        }
        crate::flash_attn_f16(
            n_tokens, n_kv, head_dim, dv, n_head, n_kv_heads, scale, softcap, bits(q), bits(k), bits(v),
            mask.map(bits), bits_mut(out),
        )
    }

    /// Attention scratch held by the engine (device bytes).
    pub fn mem_stats(&self) -> MemStats {
        crate::mem_stats()
            .map(|s| MemStats { bo_bytes: s.attention_bytes as usize, host_bytes: 0 })
            .unwrap_or_default()
    }

    pub fn trim_scratch(&mut self) {
        let _ = crate::trim_scratch();
    }

    pub fn clear_scratch(&mut self) {
        let _ = crate::clear_scratch();
    }
}
