//! The part of the `rocket-npu` driver API that code outside the extension
//! calls directly, over the MI355X library. `crates/burn-rocket` re-exports the
//! driver as `burn_rocket::npu` (lib.rs:19-20); with this crate in its place
//! (`pub use rocket_hip_sys::npu;`) these callers build unchanged:
//!
//! * Clef's expert workers: `npu::matmul::{I8Context, I8Weight}` and
//!   `npu::Error` (src/clef/engine_npu.rs:17, 63-110, 113-215, 320-345).
//!
//! `Error` and `Status` keep the driver's accessors and codes
//! (crates/rocket-npu/src/error.rs:11-175). The worker-thread counts and NPU
//! core bases of the driver contexts have no counterpart: one engine owns the
//! GPU and schedules its own work.

use std::fmt;

/// The stable failure classes (`Status`, error.rs:11-53).
#[derive(Debug, Clone, Copy, PartialEq, Eq, Hash)]
pub enum Status {
    Shape,
    Tiling,
    NoMem,
    Device,
    Unsupported,
    Range,
    Io,
}

impl Status {
    pub const fn code(self) -> i32 {
        match self {
            Status::Shape => -1,
            Status::Tiling => -2,
            Status::NoMem => -3,
            Status::Device => -4,
            Status::Unsupported => -5,
            Status::Range => -6,
            Status::Io => -7,
        }
    }

    pub const fn from_code(code: i32) -> Option<Status> {
        match code {
            -1 => Some(Status::Shape),
            -2 => Some(Status::Tiling),
            -3 => Some(Status::NoMem),
            -4 => Some(Status::Device),
            -5 => Some(Status::Unsupported),
            -6 => Some(Status::Range),
            -7 => Some(Status::Io),
            _ => None,
        }
    }
}

/// One failed operation (`Error`, error.rs:55-175): the op, its class and the
/// library's message.
#[derive(Debug, Clone)]
pub struct Error {
    op: &'static str,
    status: Status,
    detail: Option<String>,
}

impl Error {
    pub fn new(status: Status, op: &'static str, _errno: i32) -> Self {
        Self { op, status, detail: None }
    }

    pub fn shape(op: &'static str) -> Self {
        Self::new(Status::Shape, op, 0)
    }

    pub fn status(&self) -> Status {
        self.status
    }

    pub fn c_code(&self) -> i32 {
        self.status.code()
    }

    pub fn op(&self) -> &'static str {
        self.op
    }

    /// No kernel errno on this path: HIP failures carry their text in `detail`.
    pub fn errno(&self) -> i32 {
        0
    }

    pub fn detail(&self) -> Option<&str> {
        self.detail.as_deref()
    }

    pub fn is_fallback(&self) -> bool {
        matches!(self.status, Status::Shape | Status::Tiling)
    }
}

impl From<crate::Error> for Error {
    fn from(e: crate::Error) -> Self {
        Self {
            op: e.op,
            status: Status::from_code(e.rc).unwrap_or(Status::Device),
            detail: Some(crate::last_error()),
        }
    }
}

impl fmt::Display for Error {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        let what = match self.status {
            Status::Shape => "unsupported shape",
            Status::Tiling => "shape not tileable",
            Status::NoMem => "out of memory",
            Status::Device => "device failure",
            Status::Unsupported => "unsupported feature",
            Status::Range => "output out of range",
            Status::Io => "I/O failure",
        };
        write!(f, "{}: {what}", self.op)?;
        if let Some(d) = &self.detail {
            write!(f, ": {d}")?;
        }
        Ok(())
    }
}

impl std::error::Error for Error {}

pub type Result<T> = std::result::Result<T, Error>;

pub mod matmul {
    //! `I8Context` / `I8Weight` (crates/rocket-npu/src/matmul/int8.rs:112-676):
    //! resident int8 codes whose scales come with each call, the exact int32
    //! product and the group-wise scaled product on host buffers.

    use super::{Error, Result};
    use crate::WeightId;

    /// A resident int8 weight: codes only (`I8Weight`, int8.rs:112-136);
    /// group 0 is the per-channel layout.
    pub struct I8Weight {
        id: WeightId,
        m: usize,
        k: usize,
        n: usize,
        group: usize,
    }

    impl I8Weight {
        pub fn shape(&self) -> (usize, usize, usize, usize) {
            (self.m, self.k, self.n, self.group)
        }

        pub fn bytes(&self) -> usize {
            self.n * self.k
        }
    }

    /// `I8Context` (int8.rs:236-676) on the one MI355X engine.
    pub struct I8Context {
        _engine: (),
    }

    impl I8Context {
        pub fn new(_nthreads: usize) -> Result<I8Context> {
            crate::init(0)?;
            Ok(I8Context { _engine: () })
        }

        /// `new_at(nthreads, core_base)` (int8.rs:254): the NPU core base has no
        /// counterpart.
        pub fn new_at(nthreads: usize, _core_base: usize) -> Result<I8Context> {
            Self::new(nthreads)
        }

        /// The decode-shaped K-tile height of the NPU layout: nothing to set here.
        pub fn set_canonical_mt(&mut self, _mt: usize) {}

        /// Device scratch and page-locked staging of the matmul entries.
        pub fn scratch_bytes(&self) -> usize {
            crate::mem_stats()
                .map(|s| (s.scratch_bytes - s.attention_bytes + s.host_bytes) as usize)
                .unwrap_or(0)
        }

        pub fn clear_scratch(&mut self) {
            let _ = crate::clear_scratch();
        }

        fn pack(&mut self, m: usize, k: usize, n: usize, b: &[i8], group: usize) -> Result<I8Weight> {
            if b.len() != n * k || k % 32 != 0 || (group != 0 && (group % 32 != 0 || k % group != 0)) {
                return Err(Error::shape("int8/pack"));
            }
            // Per-channel codes are a group-wise weight of one K-wide group.
            let id = crate::pack_i8_codes(b, None, n, k, if group == 0 { k } else { group })?;
            Ok(I8Weight { id, m, k, n, group })
        }

        /// Per-channel codes `[N, K]` (int8.rs:450-454).
        pub fn pack_weight(&mut self, m: usize, k: usize, n: usize, b: &[i8]) -> Result<I8Weight> {
            self.pack(m, k, n, b, 0)
        }

        /// Group-wise codes `[N, K]` (int8.rs:456-472): group >= 32, group % 32 == 0, group | K.
        pub fn pack_weight_gw(&mut self, m: usize, k: usize, n: usize, b: &[i8], group: usize) -> Result<I8Weight> {
            if group == 0 {
                return Err(Error::shape("int8/pack/group"));
            }
            self.pack(m, k, n, b, group)
        }

        /// New codes for a resident weight, in place (int8.rs:474-518).
        pub fn rewrite_weight(&mut self, w: &mut I8Weight, b: &[i8]) -> Result<()> {
            if b.len() != w.n * w.k {
                return Err(Error::shape("int8/rewrite"));
            }
            Ok(crate::rewrite_i8(w.id, b, None)?)
        }

        pub fn rewrite_weight_gw(&mut self, w: &mut I8Weight, b: &[i8]) -> Result<()> {
            if w.group == 0 {
                return Err(Error::shape("int8/rewrite/group"));
            }
            self.rewrite_weight(w, b)
        }

        /// `C[M,N] = A[M,K]·B[N,K]ᵀ`, raw int32 (int8.rs:598-640); any M.
        pub fn matmul(&mut self, m: usize, k: usize, n: usize, a: &[i8], c: &mut [i32], w: &I8Weight) -> Result<()> {
            if k != w.k || n != w.n || w.group != 0 {
                return Err(Error::shape("int8/matmul/shape"));
            }
            if a.len() != m * k || c.len() != m * n {
                return Err(Error::shape("int8/matmul/buffers"));
            }
            Ok(crate::matmul_i8(w.id, a, m, k, c)?)
        }

        /// `C[M,N] = Σ_g a_scale[m,g]·b_scale[n,g]·(A_g·B_gᵀ)`, f32 (int8.rs:642-676).
        #[allow(clippy::too_many_arguments)]
        pub fn matmul_gw(
            &mut self, m: usize, k: usize, n: usize, a: &[i8], a_scale: &[f32], b_scale: &[f32], cf: &mut [f32],
            w: &I8Weight,
        ) -> Result<()> {
            if k != w.k || n != w.n || w.group == 0 {
                return Err(Error::shape("int8/matmul/shape"));
            }
            if a.len() != m * k || cf.len() != m * n {
                return Err(Error::shape("int8/matmul/buffers"));
            }
            let ng = k / w.group;
            if a_scale.len() != m * ng || b_scale.len() != n * ng {
                return Err(Error::shape("int8/matmul/scales"));
            }
            Ok(crate::matmul_i8_gw(w.id, a, a_scale, Some(b_scale), m, k, cf)?)
        }
    }
}
