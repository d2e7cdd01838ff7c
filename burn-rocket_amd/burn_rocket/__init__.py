"""Python binding of the burn-rocket MI355X op surface (libburn_rocket_amd.so).

The functions mirror the helper API of crates/burn-rocket/src/ext.rs
(`init`, `pack`, `pack2`, `pack3`, `pack_i8`, `pack_qat`, `matmul`,
`attention*`, `stats`, `mem_stats`, `trim_scratch_to`, `clear_scratch`,
ext.rs:171-308, ext.rs:561-580, ext.rs:1382-1425, ext.rs:1864-2137) over
numpy arrays, plus device-buffer plumbing for callers that keep tensors in HBM.
Every call goes through the C ABI declared in include/burn_rocket_amd.h; there
is no CPU fallback — a missing library or device raises.

Errors: a non-zero status from the library raises `RocketError` carrying the
op name and the status code (-1 shape … -7 io), as `burn_rocket::Error`
(lib.rs:119-156) does; `OpFailure` adds the m/k/n of the call (lib.rs:160-167).
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libburn_rocket_amd.so")

RK_OK = 0
RK_E_SHAPE, RK_E_TILING, RK_E_NOMEM, RK_E_DEVICE = -1, -2, -3, -4
RK_E_UNSUPPORTED, RK_E_RANGE, RK_E_IO = -5, -6, -7
RK_WEIGHT_F16, RK_WEIGHT_I8, RK_WEIGHT_QAT = 1, 2, 3
MASK_NONE, MASK_CAUSAL, MASK_WINDOW, MASK_CAUSAL_WINDOW = 0, 1, 2, 3
NOALLOC_SCRATCH_BYTES = 32 << 20  # RK_NOALLOC_SCRATCH_BYTES
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
GLU_SILU, GLU_GELU = 1, 2

# Every entry point of include/burn_rocket_amd.h with its ctypes signature.
_c = ctypes
_p, _i, _i64, _u64, _f, _sz = _c.c_void_p, _c.c_int, _c.c_int64, _c.c_uint64, _c.c_float, _c.c_size_t
SIGNATURES = {
    "rk_init": (_i, [_i]),
    "rk_last_error": (_c.c_char_p, []),
    "rk_is_fallback": (_i, [_i]),
    "rk_stats": (_i, [_p]),
    "rk_stats_reset": (_i, []),
    "rk_mem_stats": (_i, [_p]),
    "rk_trim_scratch_to": (_i, [_u64]),
    "rk_clear_scratch": (_i, []),
    "rk_trim_scratch": (_i, []),
    "rk_pack": (_i, [_p, _i64, _i64, _p]),
    "rk_pack_f16": (_i, [_p, _i64, _i64, _p]),
    "rk_pack_seg": (_i, [_p, _p, _i, _i64, _p]),
    "rk_pack_i8": (_i, [_p, _i64, _i64, _i64, _p]),
    "rk_pack_i8_codes": (_i, [_p, _p, _i64, _i64, _i64, _p]),
    "rk_rewrite_i8": (_i, [_u64, _p, _p]),
    "rk_pack_q8_0": (_i, [_p, _i64, _i64, _p]),
    "rk_pack_q8_0_f32": (_i, [_p, _i64, _i64, _p]),
    "rk_pack_qat": (_i, [_p, _p, _i64, _i64, _f, _f, _p]),
    "rk_weight_info": (_i, [_u64, _p, _p, _p, _p]),
    "rk_matmul": (_i, [_u64, _p, _i64, _i64, _p]),
    "rk_matmul_f16_dev": (_i, [_u64, _p, _i64, _i64, _p, _p]),
    "rk_matmul_f16": (_i, [_u64, _p, _i64, _i64, _p]),
    "rk_matmul_i8_gw": (_i, [_u64, _p, _p, _p, _i64, _i64, _p]),
    "rk_matmul_i8": (_i, [_u64, _p, _i64, _i64, _p]),
    "rk_pack_f16_glu": (_i, [_p, _p, _i64, _i64, _p]),
    "rk_matmul_f16_glu_dev": (_i, [_u64, _p, _i64, _i64, _i, _p, _i, _p]),
    "rk_quantize_rows_dev": (_i, [_p, _i64, _i64, _i64, _p, _p, _p]),
    "rk_matmul_w8a8_dev": (_i, [_u64, _p, _p, _i64, _i64, _i64, _p, _p]),
    "rk_matmul_w8a8_f16out_dev": (_i, [_u64, _p, _p, _i64, _i64, _i64, _p, _p]),
    "rk_matmul_i8_raw_dev": (_i, [_u64, _p, _i64, _i64, _p, _p]),
    "rk_matmul_i8_partials_dev": (_i, [_u64, _p, _i64, _i64, _p, _p]),
    "rk_attention": (_i, [_p, _p, _p, _i64, _i64, _i, _i, _i, _f, _f, _i, _i64, _i64, _i64, _p]),
    "rk_attention_dev": (_i, [_p, _p, _p, _i64, _i64, _i, _i, _i, _f, _f, _i, _i64, _i64, _i64, _p, _p]),
    "rk_attention_dev_noalloc": (_i, [_p, _p, _p, _i64, _i64, _i, _i, _i, _f, _f, _i, _i64, _i64, _i64, _p, _p]),
    "rk_flash_attn_f16": (_i, [_i64, _i64, _i, _i, _i, _i, _f, _f, _i, _i64, _i64, _i64, _p, _p, _p, _p]),
    "rk_flash_attn_f16_masked": (_i, [_i64, _i64, _i, _i, _i, _i, _f, _f, _p, _p, _p, _p, _p]),
    "rk_moe_route": (_i, [_p, _i64, _i, _i, _i, _p, _p]),
    "rk_pack_moe_q8_0": (_i, [_p, _p, _p, _i, _i64, _i64, _p]),
    "rk_pack_moe_f32": (_i, [_p, _p, _p, _i, _i64, _i64, _p]),
    "rk_moe_experts_dev": (_i, [_u64, _p, _i64, _i, _p, _p, _p, _p]),
    "rk_moe_experts_acc_dev": (_i, [_u64, _p, _i64, _i, _p, _p, _p, _p]),
    "rk_moe_plan_create": (_i, [_u64, _i64, _i, _p, _p, _p]),
    "rk_moe_experts_planned_dev": (_i, [_u64, _p, _p, _p, _p]),
    "rk_moe_experts_planned_acc_dev": (_i, [_u64, _p, _p, _p, _p]),
    "rk_moe_plan_destroy": (_i, [_p]),
    "rk_moe_gate_up_dev": (_i, [_u64, _p, _p, _p, _p]),
    "rk_device_alloc": (_i, [_sz, _p]),
    "rk_device_free": (_i, [_p]),
    "rk_memcpy_htod": (_i, [_p, _p, _sz]),
    "rk_memcpy_dtoh": (_i, [_p, _p, _sz]),
    "rk_memcpy_dtod": (_i, [_p, _p, _sz, _p]),
    "rk_silu_mul_dev": (_i, [_p, _p, _p, _i64, _i, _p]),
    "rk_gelu_mul_dev": (_i, [_p, _p, _p, _i64, _i, _p]),
    "rk_silu_mul": (_i, [_p, _p, _p, _i64]),
    "rk_pack_q8_0_glu": (_i, [_p, _p, _i64, _i64, _p]),
    "rk_pack_q8_0_glu_f32": (_i, [_p, _p, _i64, _i64, _p]),
    "rk_matmul_w8a8_glu_dev": (_i, [_u64, _p, _p, _i64, _i64, _i, _p, _i, _p]),
    "rk_gelu_mul": (_i, [_p, _p, _p, _i64]),
    "rk_rms_norm_dev": (_i, [_p, _p, _i, _p, _i64, _i64, _c.c_double, _i, _p]),
    "rk_rms_norm_noscale_dev": (_i, [_p, _p, _i64, _i64, _c.c_double, _i, _p]),
    "rk_rope_dev": (_i, [_p, _p, _p, _i, _p, _i64, _i64, _i64, _i64, _i, _p]),
    "rk_qk_norm_rope_dev": (_i, [_p, _i64, _i64, _i, _i, _i64, _p, _p, _c.c_double, _p, _p, _i,
                                 _i, _p]),
    "rk_attention_strided_dev": (_i, [_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i, _i, _i,
                                      _c.c_float, _c.c_float, _i, _i64, _i64, _i64, _p, _i64,
                                      _p]),
    "rk_attention_qkv_dev": (_i, [_p, _i64, _i64, _i, _i, _i, _p, _p, _c.c_double, _p, _p, _i,
                                  _c.c_float, _c.c_float, _i, _i64, _i64, _i64, _p, _i64, _p]),
    "rk_rms_norm_quantize_dev": (_i, [_p, _p, _i, _i64, _i64, _c.c_double, _i, _p, _p, _p]),
    "rk_rms_norm": (_i, [_p, _p, _p, _i64, _i64, _c.c_double]),
    "rk_rms_norm_noscale": (_i, [_p, _p, _i64, _i64, _c.c_double]),
    "rk_rope": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64]),
    "rk_memset_dev": (_i, [_p, _i, _sz]),
    "rk_cast_dev": (_i, [_p, _i, _p, _i, _i64, _p]),
    "rk_stream_get": (_i, [_p]),
    "rk_stream_sync": (_i, [_p]),
    "rk_stream_create": (_i, [_p]),
    "rk_stream_destroy": (_i, [_p]),
    "rk_event_create": (_i, [_p]),
    "rk_event_destroy": (_i, [_p]),
    "rk_event_record": (_i, [_p, _p]),
    "rk_event_elapsed_ms": (_i, [_p, _p, _p]),
    "rk_device_info": (_i, [_c.c_char_p, _sz, _p, _p]),
}


class RocketError(RuntimeError):
    """A failed op: `op` name and status code `rc` (lib.rs:119-156)."""

    def __init__(self, op, rc, message):
        super().__init__(message)
        self.op, self.rc = op, rc

    def is_fallback(self):
        return self.rc == RK_E_TILING


class OpFailure(RocketError):
    """A failed matmul/attention with the shape of the call (lib.rs:160-167)."""

    def __init__(self, op, rc, message, m=0, k=0, n=0):
        super().__init__(op, rc, message)
        self.m, self.k, self.n = m, k, n


_lib = None


def load_library(path=LIB_PATH):
    """Load the C-ABI library (no initialisation, no device access)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RocketError("load", RK_E_IO, f"{path} is missing: run burn-rocket_amd/build.py")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    _lib = lib
    return lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _check(rc, op, m=0, k=0, n=0):
    if rc != RK_OK:
        msg = _lib.rk_last_error().decode()
        raise OpFailure(op, rc, msg or f"{op} failed (rc={rc})", m, k, n)


def init(device=0):
    """Create the global engine (`burn_rocket::init`, ext.rs:561-580)."""
    lib = load_library()
    _check(lib.rk_init(device), "rk_init")


class WeightId(int):
    """Registry id of a resident weight (`WeightId`, ext.rs:39-51)."""

    def id(self):
        return int(self)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def pack(w):
    """Resident fp16 weight from an [N, K] f32/f16 array (`pack`, ext.rs:1866)."""
    w = np.asarray(w)
    assert w.ndim == 2, "weights are [N, K]"
    n, k = w.shape
    out = ctypes.c_uint64()
    if w.dtype == np.float16:
        w16 = np.ascontiguousarray(w).view(np.uint16)
        _check(_lib.rk_pack_f16(_ptr(w16), n, k, ctypes.byref(out)), "rocket_weights_pack", 0, k, n)
    else:
        wf = _f32(w)
        _check(_lib.rk_pack(_ptr(wf), n, k, ctypes.byref(out)), "rocket_weights_pack", 0, k, n)
    return WeightId(out.value)


def _pack_many(parts):
    parts = [_f32(p) for p in parts]
    k = parts[0].shape[1]
    assert all(p.ndim == 2 and p.shape[1] == k for p in parts), "all parts must share K"
    ptrs = (ctypes.c_void_p * len(parts))(*[p.ctypes.data for p in parts])
    ns = (ctypes.c_int64 * len(parts))(*[p.shape[0] for p in parts])
    out = ctypes.c_uint64()
    _check(_lib.rk_pack_seg(ctypes.cast(ptrs, ctypes.c_void_p), ctypes.cast(ns, ctypes.c_void_p),
                            len(parts), k, ctypes.byref(out)), "rocket_weights_pack_seg")
    return WeightId(out.value)


def pack2(a, b):
    """Two weights sharing one input, concatenated along N (ext.rs:1870)."""
    return _pack_many([a, b])


def pack3(a, b, c):
    """Three weights sharing one input, concatenated along N (ext.rs:1879)."""
    return _pack_many([a, b, c])


def pack_i8(w, group):
    """Resident group-wise int8 weight (`pack_i8`, ext.rs:1892)."""
    wf = _f32(w)
    n, k = wf.shape
    assert group > 0 and group % 32 == 0 and k % group == 0, \
        f"int8 group {group} must be a positive multiple of 32 dividing K={k}"
    out = ctypes.c_uint64()
    _check(_lib.rk_pack_i8(_ptr(wf), n, k, group, ctypes.byref(out)), "rocket_i8_weights_pack_gw", 0, k, n)
    return WeightId(out.value)


def pack_i8_codes(codes, scales, group):
    """Pre-quantized group-wise weight; scales None keeps the codes alone
    (`I8Context::pack_weight_gw`: the scales come with each matmul_gw)."""
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    scales = None if scales is None else _f32(scales)
    n, k = codes.shape
    out = ctypes.c_uint64()
    _check(_lib.rk_pack_i8_codes(_ptr(codes), None if scales is None else _ptr(scales), n, k, group,
                                 ctypes.byref(out)),
           "rocket_i8_weights_pack_gw", 0, k, n)
    return WeightId(out.value)


def rewrite_i8(wid, codes, scales=None):
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    scales = None if scales is None else _f32(scales)
    _check(_lib.rk_rewrite_i8(int(wid), _ptr(codes), None if scales is None else _ptr(scales)),
           "rocket_i8_rewrite_gw")


def pack_q8_0(blocks, n, k):
    """Resident weight from GGUF Q8_0 blocks (34 bytes per 32 values)."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    assert blocks.size == n * (k // 32) * 34, "Q8_0 blob size"
    out = ctypes.c_uint64()
    _check(_lib.rk_pack_q8_0(_ptr(blocks), n, k, ctypes.byref(out)), "rocket_q8_0_pack", 0, k, n)
    return WeightId(out.value)


def pack_q8_0_glu(gate_blocks, up_blocks, n, k):
    """Fused gate|up weight from the GGUF Q8_0 blocks of gate [n, k] and up [n, k]."""
    g = np.ascontiguousarray(gate_blocks, dtype=np.uint8)
    u = np.ascontiguousarray(up_blocks, dtype=np.uint8)
    assert g.size == n * (k // 32) * 34 and u.size == g.size, "Q8_0 blob size"
    out = ctypes.c_uint64()
    _check(_lib.rk_pack_q8_0_glu(_ptr(g), _ptr(u), n, k, ctypes.byref(out)), "rocket_q8_0_glu_pack", 0, k, n)
    return WeightId(out.value)


def pack_q8_0_glu_f32(gate, up):
    """Fused gate|up weight quantized to Q8_0 on the device from f32 gate, up [n, k]."""
    g, u = _f32(gate), _f32(up)
    assert g.shape == u.shape and g.ndim == 2
    n, k = g.shape
    out = ctypes.c_uint64()
    _check(_lib.rk_pack_q8_0_glu_f32(_ptr(g), _ptr(u), n, k, ctypes.byref(out)), "rocket_q8_0_glu_pack", 0, k, n)
    return WeightId(out.value)


def pack_f16_glu(gate, up):
    """fp16 gate|up weight for rk_matmul_f16_glu_dev from f32 gate, up [n, k]."""
    g, u = _f32(gate), _f32(up)
    assert g.shape == u.shape and g.ndim == 2
    n, k = g.shape
    out = ctypes.c_uint64()
    _check(_lib.rk_pack_f16_glu(_ptr(g), _ptr(u), n, k, ctypes.byref(out)), "rocket_weights_pack_glu", 0, k, n)
    return WeightId(out.value)


def pack_q8_0_f32(w):
    """Resident Q8_0 weight quantized on the device from f32 [N, K]."""
    wf = _f32(w)
    n, k = wf.shape
    out = ctypes.c_uint64()
    _check(_lib.rk_pack_q8_0_f32(_ptr(wf), n, k, ctypes.byref(out)), "rocket_q8_0_pack", 0, k, n)
    return WeightId(out.value)


def pack_qat(codes, w_scale, n, k, in_scale, out_scale):
    """Per-channel QAT weight (`pack_qat`, ext.rs:1382-1425)."""
    codes = np.ascontiguousarray(codes, dtype=np.int8).reshape(n, k)
    w_scale = _f32(w_scale)
    assert w_scale.size == n, "one weight scale per output channel"
    assert in_scale >= 0.0, "QAT input scale must not be negative"
    out = ctypes.c_uint64()
    _check(_lib.rk_pack_qat(_ptr(codes), _ptr(w_scale), n, k, in_scale, out_scale, ctypes.byref(out)),
           "rocket_i8_weights_pack", 0, k, n)
    return WeightId(out.value)


def weight_info(wid):
    kind, n, k, g = ctypes.c_int(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    _check(_lib.rk_weight_info(int(wid), ctypes.byref(kind), ctypes.byref(n), ctypes.byref(k), ctypes.byref(g)),
           "weight_info")
    return kind.value, n.value, k.value, g.value


def matmul(x, wid):
    """`x[.., M, K] @ W[N, K]ᵀ -> [.., M, N]` (`matmul`, ext.rs:1900); f32 in/out."""
    x = np.asarray(x)
    assert x.ndim >= 2, "matmul needs at least [M, K]"
    k = x.shape[-1]
    m = int(np.prod(x.shape[:-1]))
    _, n, wk, _ = weight_info(wid)
    assert wk == k, f"activation K mismatch for weight id {int(wid)}"
    xf = _f32(x).reshape(m, k)
    y = np.empty((m, n), dtype=np.float32)
    _check(_lib.rk_matmul(int(wid), _ptr(xf), m, k, _ptr(y)), "rocket_matmul", m, k, n)
    return y.reshape(*x.shape[:-1], n).astype(x.dtype if x.dtype in (np.float16, np.float32) else np.float32)


def _glue(fn_name, op_name, a, b, bf16):
    a, b = np.asarray(a), np.asarray(b)
    assert a.dtype == b.dtype, f"{op_name} inputs must share a dtype"
    assert a.shape == b.shape, f"{op_name} inputs must share a shape"
    if bf16:
        assert a.dtype == np.uint16, "bf16 values are passed as their uint16 bits"
        dt = DTYPE_BF16
    elif a.dtype == np.float16:
        dt = DTYPE_F16
    elif a.dtype == np.float32:
        dt = DTYPE_F32
    else:
        raise AssertionError(f"unsupported glue dtype {a.dtype} (f32/f16/bf16)")
    if a.size == 0:
        return a.copy()
    ac, bc = np.ascontiguousarray(a), np.ascontiguousarray(b)
    da, db = DeviceBuffer.from_array(ac), DeviceBuffer.from_array(bc)
    do = DeviceBuffer(max(ac.nbytes, 1))
    try:
        _check(getattr(_lib, fn_name)(da.ptr, db.ptr, do.ptr, ac.size, dt, None), op_name)
        synchronize()
        return do.download(a.shape, a.dtype)
    finally:
        for buf in (da, db, do):
            buf.free()


def silu_mul(a, b, bf16=False):
    """`silu(a) * b` (`rocket_silu_mul`, ext.rs:607-608): f32 or f16 arrays, or
    bf16 as uint16 bits with bf16=True; computed in f32, returned in the input
    dtype."""
    return _glue("rk_silu_mul_dev", "rocket_silu_mul", a, b, bf16)


def gelu_mul(a, b, bf16=False):
    """`gelu_approximate(a) * b` (`rocket_gelu_mul`, ext.rs:603-604); as silu_mul."""
    return _glue("rk_gelu_mul_dev", "rocket_gelu_mul", a, b, bf16)


def _float_dtype(a, bf16, op_name):
    if bf16:
        assert a.dtype == np.uint16, "bf16 values are passed as their uint16 bits"
        return DTYPE_BF16
    if a.dtype == np.float16:
        return DTYPE_F16
    if a.dtype == np.float32:
        return DTYPE_F32
    raise AssertionError(f"unsupported {op_name} dtype {a.dtype} (f32/f16/bf16)")


def _run_dev(fn_name, op_name, out_like, inputs, build_args):
    """Upload `inputs`, call `fn_name` with build_args(device pointers, out pointer),
    return the output shaped and typed like out_like."""
    bufs = [DeviceBuffer.from_array(np.ascontiguousarray(a)) for a in inputs]
    do = DeviceBuffer(max(out_like.nbytes, 1))
    try:
        _check(getattr(_lib, fn_name)(*build_args([b.ptr for b in bufs], do.ptr)), op_name)
        synchronize()
        return do.download(out_like.shape, out_like.dtype)
    finally:
        for buf in bufs + [do]:
            buf.free()


def rms_norm(x, w, eps, bf16=False):
    """Weighted RMSNorm over the last dim, `x * (mean(x^2) + eps)^-0.5 * w`
    (`burn_rocket::rms_norm`, ext.rs:2112-2119): x f32/f16 (or bf16 bits with
    bf16=True), w [D] of the same type; computed in f32, returned in x's type."""
    x, w = np.asarray(x), np.asarray(w)
    dt = _float_dtype(x, bf16, "rocket_rms_norm")
    assert x.ndim >= 1, "rms_norm needs at least one dim"
    d = x.shape[-1]
    assert w.shape == (d,) and w.dtype == x.dtype, "rms_norm: the weight has the last dim's size"
    if x.size == 0:
        return x.copy()
    return _run_dev("rk_rms_norm_dev", "rocket_rms_norm", x, [x, w],
                    lambda p, o: (p[0], p[1], dt, o, x.size // d, d, float(eps), dt, None))


def rms_norm_noscale(x, eps, bf16=False):
    """Scale-free RMSNorm over the last dim (`burn_rocket::rms_norm_noscale`,
    ext.rs:2121-2128); as rms_norm."""
    x = np.asarray(x)
    dt = _float_dtype(x, bf16, "rocket_rms_norm_noscale")
    d = x.shape[-1]
    if x.size == 0:
        return x.copy()
    return _run_dev("rk_rms_norm_noscale_dev", "rocket_rms_norm_noscale", x, [x],
                    lambda p, o: (p[0], o, x.size // d, d, float(eps), dt, None))


def rope_apply(x, cos, sin, bf16=False):
    """Rotate-half RoPE (`burn_rocket::rope_apply`, ext.rs:2130-2137): x
    [B, S, H, D], cos/sin [S, D/2] of x's type; returned in x's type."""
    x, cos, sin = np.asarray(x), np.asarray(cos), np.asarray(sin)
    dt = _float_dtype(x, bf16, "rocket_rope")
    assert x.ndim == 4, "rope: x must be [B, S, H, D]"
    b, s, h, d = x.shape
    assert d % 2 == 0, "rope: the head dim must be even"
    assert cos.shape == (s, d // 2) and cos.dtype == x.dtype, "rope: cos must be [S, D/2]"
    assert sin.shape == (s, d // 2) and sin.dtype == x.dtype, "rope: sin must be [S, D/2]"
    if x.size == 0:
        return x.copy()
    return _run_dev("rk_rope_dev", "rocket_rope", x, [x, cos, sin],
                    lambda p, o: (p[0], p[1], p[2], dt, o, b, s, h, d, dt, None))


def _attention(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, mode, window, q0, k0):
    q, k, v = np.asarray(q), np.asarray(k), np.asarray(v)
    assert q.ndim == 3 and q.shape[0] == 1, "attention input must be [1, S, H*D] (batch 1)"
    assert q.shape[2] == n_head * head_dim, "q width must be n_head * head_dim"
    n, n_k = q.shape[1], k.shape[1]
    assert k.shape == (1, n_k, n_kv_heads * head_dim), "k must be [1, S, KV*D]"
    assert v.shape == (1, n_k, n_kv_heads * head_dim), "v must be [1, S, KV*D]"
    out = np.empty((n, n_head * head_dim), dtype=np.float32)
    qf, kf, vf = _f32(q[0]), _f32(k[0]), _f32(v[0])
    _check(_lib.rk_attention(_ptr(qf), _ptr(kf), _ptr(vf), n, n_k, n_head, n_kv_heads, head_dim,
                             float(scale), float(softcap or 0.0), mode, window, q0, k0, _ptr(out)),
           "rocket_flash_attn_fp16_ctx", n, n_k, head_dim)
    return out.reshape(1, n, n_head * head_dim).astype(q.dtype if q.dtype == np.float16 else np.float32)


def attention(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap=None, is_causal=False):
    """Masked GQA attention (`attention`, ext.rs:1910)."""
    mode = MASK_CAUSAL if is_causal else MASK_NONE
    return _attention(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, mode, -1, 0, 0)


def attention_window(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, window):
    """|t - j| <= window, window < 0 = no mask (ext.rs:1938)."""
    return _attention(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, MASK_WINDOW, window, 0, 0)


def attention_causal_window(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, window):
    """t - window < j <= t, window < 0 = causal (ext.rs:1966)."""
    return _attention(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, MASK_CAUSAL_WINDOW, window, 0, 0)


def attention_window_block(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, window, q_start, kv_start):
    """Band over a query chunk at absolute offsets (ext.rs:1996)."""
    return _attention(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, MASK_WINDOW, window, q_start,
                      kv_start)


def attention_causal_block(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, q_start, kv_start):
    """Causal over a query chunk at absolute offsets (ext.rs:2034)."""
    return _attention(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, MASK_CAUSAL, -1, q_start,
                      kv_start)


def attention_causal_block_window(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, window, q_start,
                                  kv_start):
    """Causal sliding window over a query chunk (ext.rs:2068)."""
    return _attention(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, MASK_CAUSAL_WINDOW, window,
                      q_start, kv_start)


def flash_attn_f16(q, k, v, n_q, n_kv, head_dim, n_head, n_kv_heads, scale, softcap=0.0, mode=MASK_NONE,
                   window=-1, q0=0, k0=0, dv=None):
    """Head-major fp16 attention (`RocketFaCtx::flash_attn`, lib.rs:294-323):
    q [H][n_q][head_dim], k [KV][n_kv][head_dim], v [KV][dv][n_kv] →
    out [H][n_q][dv] (fp16); dv defaults to head_dim."""
    dv = head_dim if dv is None else dv
    q16 = np.ascontiguousarray(q, dtype=np.float16).view(np.uint16)
    k16 = np.ascontiguousarray(k, dtype=np.float16).view(np.uint16)
    v16 = np.ascontiguousarray(v, dtype=np.float16).view(np.uint16)
    assert q16.size >= n_head * n_q * head_dim and k16.size >= n_kv_heads * n_kv * head_dim, "flash_attn/buffers"
    assert v16.size >= n_kv_heads * dv * n_kv, "flash_attn/buffers"
    out = np.empty(n_head * n_q * dv, dtype=np.uint16)
    _check(_lib.rk_flash_attn_f16(n_q, n_kv, head_dim, dv, n_head, n_kv_heads, float(scale),
                                  float(softcap), mode, window, q0, k0, _ptr(q16), _ptr(k16), _ptr(v16),
                                  _ptr(out)), "rocket_flash_attn_fp16_ctx", n_q, n_kv, head_dim)
    return out.view(np.float16).reshape(n_head, n_q, dv)


def moe_route(logits, top_k, norm_topk=True):
    """Router top-k (`route`, src/clef/model.rs:462-489): ids [s, k], weights [s, k]."""
    logits = _f32(logits)
    s, e = logits.shape
    ids = np.empty((s, top_k), dtype=np.uint32)
    wts = np.empty((s, top_k), dtype=np.float32)
    _check(_lib.rk_moe_route(_ptr(logits), s, e, top_k, int(norm_topk), _ptr(ids), _ptr(wts)), "route")
    return ids, wts


def pack_moe_q8_0(gate_blocks, up_blocks, down_blocks, n_experts, hidden, inter):
    g = np.ascontiguousarray(gate_blocks, dtype=np.uint8)
    u = np.ascontiguousarray(up_blocks, dtype=np.uint8)
    d = np.ascontiguousarray(down_blocks, dtype=np.uint8)
    out = ctypes.c_uint64()
    _check(_lib.rk_pack_moe_q8_0(_ptr(g), _ptr(u), _ptr(d), n_experts, hidden, inter, ctypes.byref(out)),
           "pack_moe")
    return WeightId(out.value)


def pack_moe_f32(gate, up, down):
    """Expert stack from f32 gate/up [E, I, H] and down [E, H, I], Q8_0 on device."""
    g, u, d = _f32(gate), _f32(up), _f32(down)
    E, I, H = g.shape
    assert u.shape == (E, I, H) and d.shape == (E, H, I)
    out = ctypes.c_uint64()
    _check(_lib.rk_pack_moe_f32(_ptr(g), _ptr(u), _ptr(d), E, H, I, ctypes.byref(out)), "pack_moe")
    return WeightId(out.value)


class Stats(ctypes.Structure):
    """`burn_rocket::Stats` (ext.rs:175-183): conversion and device seconds of the
    host-buffer ops, and the matmul / attention / MoE call count."""
    _fields_ = [("convert_s", ctypes.c_double), ("npu_s", ctypes.c_double), ("calls", ctypes.c_uint64)]


class MemStats(ctypes.Structure):
    """`rk_mem_stats_t`: resident weights, device scratch (all / attention),
    page-locked staging bytes (`MemStats`, lib.rs:44-84)."""
    _fields_ = [("weights_bytes", ctypes.c_uint64), ("scratch_bytes", ctypes.c_uint64),
                ("n_weights", ctypes.c_uint64), ("attention_bytes", ctypes.c_uint64),
                ("host_bytes", ctypes.c_uint64), ("n_scratch", ctypes.c_uint64)]


def stats():
    s = Stats()
    _check(_lib.rk_stats(ctypes.byref(s)), "stats")
    return s


def stats_reset():
    _check(_lib.rk_stats_reset(), "stats_reset")


def mem_stats():
    s = MemStats()
    _check(_lib.rk_mem_stats(ctypes.byref(s)), "mem_stats")
    return s


def trim_scratch_to(budget):
    _check(_lib.rk_trim_scratch_to(int(budget)), "trim_scratch_to")


def clear_scratch():
    _check(_lib.rk_clear_scratch(), "clear_scratch")


def trim_scratch():
    """`burn_rocket::trim_scratch` (ext.rs:254-265): scratch unused since the
    previous trim is freed; the just-used set stays."""
    _check(_lib.rk_trim_scratch(), "trim_scratch")


def _shape_error(op, what):
    raise RocketError(op, RK_E_SHAPE, f"{op} failed: unsupported shape (rc=-1): {what}")


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.float16).view(np.uint16)


class RocketWeight:
    """A resident fp16 weight of a `RocketCtx` (`RocketWeight`, lib.rs:268-270)."""

    def __init__(self, wid, m, k, n):
        self.id, self.m, self.k, self.n = WeightId(wid), m, k, n

    def bytes(self):
        return self.n * self.k * 2


class RocketCtx:
    """`burn_rocket::RocketCtx` (lib.rs:203-266): resident fp16 weights and
    `C[M, N] = A[M, K]·B[N, K]ᵀ` on host fp16 buffers. `nthreads` (the NPU
    worker count) has no counterpart; scratch belongs to the one engine."""

    def __init__(self, nthreads=1):
        init(0)

    def pack_weight(self, m, k, n, b):
        b = _u16(b)
        if b.size != n * k:
            _shape_error("rocket_weights_pack", "b must be [N, K]")
        out = ctypes.c_uint64()
        _check(_lib.rk_pack_f16(_ptr(b), n, k, ctypes.byref(out)), "rocket_weights_pack", m, k, n)
        return RocketWeight(out.value, m, k, n)

    def pack_weight_seg(self, m, k, parts):
        parts = [np.ascontiguousarray(p, dtype=np.float16).ravel() for p in parts]
        if any(p.size % k for p in parts):
            _shape_error("rocket_weights_pack_seg", "every part must be [n_i, K]")
        return self.pack_weight(m, k, sum(p.size // k for p in parts), np.concatenate(parts))

    def matmul_prepacked(self, m, k, n, a, c, w):
        """Fills the fp16 array `c` [M·N] in place."""
        a = _u16(a)
        if k != w.k or n != w.n or a.size != m * k or c.size != m * n or c.dtype != np.float16:
            _shape_error("rocket_matmul_fp16", "A [M, K], C [M, N] fp16 and the weight's K, N")
        out = np.empty(m * n, dtype=np.uint16)
        _check(_lib.rk_matmul_f16(int(w.id), _ptr(a), m, k, _ptr(out)), "rocket_matmul_fp16", m, k, n)
        c.reshape(-1)[:] = out.view(np.float16)

    def trim_scratch(self):
        trim_scratch()

    def trim_to_budget(self, budget):
        trim_scratch_to(budget)

    def scratch_bytes(self):
        ms = mem_stats()
        return ms.scratch_bytes - ms.attention_bytes + ms.host_bytes

    def clear_scratch(self):
        clear_scratch()


class RocketFaCtx:
    """`burn_rocket::RocketFaCtx` (lib.rs:285-330): head-major fp16 masked GQA
    attention, q [H][T][head_dim], k [KV][Nk][head_dim], v [KV][dv][Nk],
    out [H][T][dv], optional additive fp16 mask [T][Nk] of 0 / -inf."""

    def __init__(self, nthreads=1):
        init(0)

    def flash_attn(self, n_tokens, n_kv, head_dim, dv, n_head, n_kv_heads, scale, softcap, q, k, v, mask, out):
        q16, k16, v16 = _u16(q), _u16(k), _u16(v)
        if (q16.size != n_head * n_tokens * head_dim or k16.size != n_kv_heads * n_kv * head_dim
                or v16.size != n_kv_heads * dv * n_kv or out.size != n_head * n_tokens * dv
                or out.dtype != np.float16):
            _shape_error("rocket_flash_attn_fp16_ctx", "q, k, v or out do not match the shapes")
        m16 = None
        if mask is not None:
            m16 = _u16(mask)
            if m16.size != n_tokens * n_kv:
                _shape_error("rocket_flash_attn_fp16_ctx", "mask must be [n_tokens, n_kv]")
        o = np.empty(n_head * n_tokens * dv, dtype=np.uint16)
        _check(_lib.rk_flash_attn_f16_masked(n_tokens, n_kv, head_dim, dv, n_head, n_kv_heads, float(scale),
                                             float(softcap), None if m16 is None else _ptr(m16), _ptr(q16),
                                             _ptr(k16), _ptr(v16), _ptr(o)),
               "rocket_flash_attn_fp16_ctx", n_tokens, n_kv, head_dim)
        out.reshape(-1)[:] = o.view(np.float16)

    def mem_stats(self):
        ms = mem_stats()
        return {"bo_bytes": ms.attention_bytes, "host_bytes": 0}

    def trim_scratch(self):
        trim_scratch()

    def clear_scratch(self):
        clear_scratch()


class I8Weight:
    """A resident int8 weight of an `I8Context` (int8.rs:112-136): codes only;
    group 0 is the per-channel layout."""

    def __init__(self, wid, m, k, n, group):
        self.id, self.m, self.k, self.n, self.group = WeightId(wid), m, k, n, group

    def shape(self):
        return self.m, self.k, self.n, self.group

    def bytes(self):
        return self.n * self.k


class I8Context:
    """`rocket_npu::matmul::I8Context` (int8.rs:236-676) as Clef's expert
    workers use it (src/clef/engine_npu.rs:75-207): resident int8 codes whose
    scales come with each call, exact int32 products and the group-wise
    scaled product on host buffers. The worker count and core base of the NPU
    have no counterpart."""

    def __init__(self, nthreads=1, core_base=0):
        init(0)

    @classmethod
    def new_at(cls, nthreads, core_base):
        return cls(nthreads, core_base)

    def _pack(self, m, k, n, b, group, op):
        b = np.ascontiguousarray(b, dtype=np.int8)
        if b.size != n * k:
            _shape_error(op, "b must be [N, K] int8")
        out = ctypes.c_uint64()
        _check(_lib.rk_pack_i8_codes(_ptr(b), None, n, k, group if group else k, ctypes.byref(out)), op, m, k, n)
        return I8Weight(out.value, m, k, n, group)

    def pack_weight(self, m, k, n, b):
        return self._pack(m, k, n, b, 0, "rocket_i8_weights_pack")

    def pack_weight_gw(self, m, k, n, b, group):
        if group == 0:
            _shape_error("int8/pack/group", "group-wise weight needs group > 0")
        return self._pack(m, k, n, b, group, "rocket_i8_weights_pack_gw")

    def rewrite_weight(self, w, b):
        b = np.ascontiguousarray(b, dtype=np.int8)
        if b.size != w.n * w.k:
            _shape_error("int8/rewrite", "b must be [N, K] int8")
        _check(_lib.rk_rewrite_i8(int(w.id), _ptr(b), None), "int8/rewrite")

    def rewrite_weight_gw(self, w, b):
        if w.group == 0:
            _shape_error("int8/rewrite/group", "the weight is per-channel")
        self.rewrite_weight(w, b)

    def matmul(self, m, k, n, a, c, w):
        """Raw int32 product into `c` [M·N] (int32)."""
        a = np.ascontiguousarray(a, dtype=np.int8)
        if k != w.k or n != w.n or w.group != 0:
            _shape_error("int8/matmul/shape", "per-channel weight of this K, N")
        if a.size != m * k or c.size != m * n or c.dtype != np.int32:
            _shape_error("int8/matmul/buffers", "a [M, K] int8, c [M, N] int32")
        out = np.empty(m * n, dtype=np.int32)
        _check(_lib.rk_matmul_i8(int(w.id), _ptr(a), m, k, _ptr(out)), "rocket_matmul_int8_prepacked", m, k, n)
        c.reshape(-1)[:] = out

    def matmul_gw(self, m, k, n, a, a_scale, b_scale, cf, w):
        """`cf[m, n] = Σ_g a_scale[m,g]·b_scale[n,g]·(A_g·B_gᵀ)` into `cf` (f32)."""
        a = np.ascontiguousarray(a, dtype=np.int8)
        if k != w.k or n != w.n or w.group == 0:
            _shape_error("int8/matmul/shape", "group-wise weight of this K, N")
        if a.size != m * k or cf.size != m * n or cf.dtype != np.float32:
            _shape_error("int8/matmul/buffers", "a [M, K] int8, cf [M, N] f32")
        ng = k // w.group
        a_scale, b_scale = _f32(a_scale), _f32(b_scale)
        if a_scale.size != m * ng or b_scale.size != n * ng:
            _shape_error("int8/matmul/scales", "a_scale [M, K/group], b_scale [N, K/group]")
        out = np.empty(m * n, dtype=np.float32)
        _check(_lib.rk_matmul_i8_gw(int(w.id), _ptr(a), _ptr(a_scale), _ptr(b_scale), m, k, _ptr(out)),
               "rocket_matmul_int8_prepacked_gw", m, k, n)
        cf.reshape(-1)[:] = out

    def scratch_bytes(self):
        ms = mem_stats()
        return ms.scratch_bytes - ms.attention_bytes + ms.host_bytes

    def clear_scratch(self):
        clear_scratch()


# ------------------------------------------------------------- device buffers
class DeviceBuffer:
    """Device memory owned through the library (no torch, one HIP runtime)."""

    def __init__(self, nbytes):
        p = ctypes.c_void_p()
        _check(_lib.rk_device_alloc(int(nbytes), ctypes.byref(p)), "device_alloc")
        self.ptr, self.nbytes = p.value, int(nbytes)

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _check(_lib.rk_memcpy_htod(ctypes.c_void_p(self.ptr), _ptr(a), a.nbytes), "memcpy_htod")

    def download(self, shape, dtype):
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        _check(_lib.rk_memcpy_dtoh(_ptr(out), ctypes.c_void_p(self.ptr), out.nbytes), "memcpy_dtoh")
        return out

    def zero(self):
        _check(_lib.rk_memset_dev(ctypes.c_void_p(self.ptr), 0, self.nbytes), "memset")

    def free(self):
        if self.ptr:
            _check(_lib.rk_device_free(ctypes.c_void_p(self.ptr)), "device_free")
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.rk_device_free(ctypes.c_void_p(self.ptr))
        except Exception:
            pass


def stream():
    s = ctypes.c_void_p()
    _check(_lib.rk_stream_get(ctypes.byref(s)), "stream_get")
    return s.value


def new_stream():
    """A new HIP stream (default priority) owned by the caller; free with destroy_stream."""
    s = ctypes.c_void_p()
    _check(_lib.rk_stream_create(ctypes.byref(s)), "stream_create")
    return s.value


def destroy_stream(st):
    _check(_lib.rk_stream_destroy(ctypes.c_void_p(st)), "stream_destroy")


def synchronize(st=None):
    _check(_lib.rk_stream_sync(ctypes.c_void_p(st) if st else None), "stream_sync")


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        _check(_lib.rk_event_create(ctypes.byref(e)), "event_create")
        self.ptr = e.value

    def record(self, st=None):
        _check(_lib.rk_event_record(ctypes.c_void_p(self.ptr), ctypes.c_void_p(st) if st else None),
               "event_record")

    def elapsed_ms(self, end):
        ms = ctypes.c_float()
        _check(_lib.rk_event_elapsed_ms(ctypes.c_void_p(self.ptr), ctypes.c_void_p(end.ptr),
                                        ctypes.byref(ms)), "event_elapsed")
        return ms.value


def device_info():
    name = ctypes.create_string_buffer(256)
    cus, clk = ctypes.c_int(), ctypes.c_int()
    _check(_lib.rk_device_info(name, 256, ctypes.byref(cus), ctypes.byref(clk)), "device_info")
    return name.value.decode(), cus.value, clk.value


def lib():
    return load_library()
