"""ctypes wrapper of the CPU oracle (oracle/liboracle.so) and parity metrics.

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the parity reference or the timed CPU baseline. The
functions restate the reference (see oracle.c for file:line citations).
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_c = ctypes
_p, _i, _i64, _f = _c.c_void_p, _c.c_int, _c.c_int64, _c.c_float
_SIG = {
    "orc_f32_to_f16": (_c.c_uint16, [_f]),
    "orc_f16_to_f32": (_f, [_c.c_uint16]),
    "orc_f32_to_f16_vec": (None, [_p, _p, _i64]),
    "orc_f16_to_f32_vec": (None, [_p, _p, _i64]),
    "orc_gemm_f16": (None, [_p, _p, _i64, _i64, _i64, _p, _i]),
    "orc_gemm_f16_f64": (None, [_p, _p, _i64, _i64, _i64, _p, _i]),
    "orc_quantize_row_groups": (None, [_p, _i64, _i64, _p, _p]),
    "orc_quantize_rows": (None, [_p, _i64, _i64, _i64, _p, _p, _i]),
    "orc_q8_0_quantize": (None, [_p, _i64, _i64, _p, _p]),
    "orc_q8_0_to_blocks": (None, [_p, _p, _i64, _i64, _p]),
    "orc_q8_0_dequant": (None, [_p, _i64, _p]),
    "orc_quantize_static": (None, [_p, _i64, _i64, _f, _p, _p]),
    "orc_qat_epilogue": (None, [_p, _p, _p, _i64, _i64, _f, _p]),
    "orc_matmul_i8_raw": (None, [_p, _p, _i64, _i64, _i64, _p, _i]),
    "orc_i8_block_partials": (None, [_p, _p, _i64, _i64, _i64, _p, _i]),
    "orc_emu_matmul_gw": (None, [_p, _p, _i64, _i64, _i64, _p, _p, _i64, _i64, _p, _i]),
    "orc_mask_keep": (_i, [_i, _i64, _i64, _i64]),
    "orc_attention_ref": (None, [_p, _p, _p, _i64, _i64, _i, _i, _i, _f, _f, _i, _i64, _i64, _i64, _p, _i]),
    "orc_attention_flex": (None, [_p, _p, _p, _i64, _i64, _i, _i, _i, _f, _f, _i, _i64, _i64, _i64, _p, _i]),
    "orc_route": (None, [_p, _i64, _i, _i, _i, _p, _p]),
    "orc_moe_experts": (None, [_p, _i64, _i64, _i64, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i]),
    "orc_gelu_tanh": (_f, [_f]),
    "orc_gelu_mul": (None, [_p, _p, _p, _i64]),
    "orc_silu_mul": (None, [_p, _p, _p, _i64]),
    "orc_clef_silu_mul": (None, [_p, _p, _p, _i64]),
    "orc_rms_norm": (None, [_p, _p, _p, _i64, _i64, _c.c_float]),
    "orc_rope": (None, [_p, _p, _p, _p, _i64, _i64, _i64, _i64]),
    "orc_max_threads": (_i, []),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIG.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def threads_default():
    return max(1, min(16, os.cpu_count() or 1))


# ---------------------------------------------------------------- fp16 ----
def f32_to_f16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_vec(_ptr(x), _ptr(y), x.size)
    return y


def f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32_vec(_ptr(h), _ptr(y), h.size)
    return y


def _u16(a):
    a = np.asarray(a)
    if a.dtype == np.float16:
        return np.ascontiguousarray(a).view(np.uint16)
    return np.ascontiguousarray(a, dtype=np.uint16)


# ---------------------------------------------------------------- GEMM ----
def gemm_f16(a, b, threads=None):
    """a f16 [m,k], b f16 [n,k] → f32 [m,n] (f32 accumulation)."""
    a, b = _u16(a), _u16(b)
    m, k = a.shape
    n = b.shape[0]
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_gemm_f16(_ptr(a), _ptr(b), m, n, k, _ptr(c), threads or threads_default())
    return c


def gemm_f16_f64(a, b, threads=None):
    a, b = _u16(a), _u16(b)
    m, k = a.shape
    n = b.shape[0]
    c = np.empty((m, n), dtype=np.float64)
    lib().orc_gemm_f16_f64(_ptr(a), _ptr(b), m, n, k, _ptr(c), threads or threads_default())
    return c


# ---------------------------------------------------------- quantizers ----
def quantize_rows(x, group, threads=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    q = np.empty((m, k), dtype=np.int8)
    s = np.empty((m, k // group), dtype=np.float32)
    lib().orc_quantize_rows(_ptr(x), m, k, group, _ptr(q), _ptr(s), threads or threads_default())
    return q, s


def q8_0_quantize(w):
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    q = np.empty((n, k), dtype=np.int8)
    d = np.empty((n, k // 32), dtype=np.uint16)
    lib().orc_q8_0_quantize(_ptr(w), n, k, _ptr(q), _ptr(d))
    return q, d


def q8_0_blocks(q, d16):
    q = np.ascontiguousarray(q, dtype=np.int8)
    d16 = np.ascontiguousarray(d16, dtype=np.uint16)
    n, k = q.shape
    blocks = np.empty(n * (k // 32) * 34, dtype=np.uint8)
    lib().orc_q8_0_to_blocks(_ptr(q), _ptr(d16), n, k, _ptr(blocks))
    return blocks


def q8_0_dequant(blocks, nvals):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(nvals, dtype=np.float32)
    lib().orc_q8_0_dequant(_ptr(blocks), nvals, _ptr(out))
    return out


def quantize_static(x, in_scale):
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    q = np.empty((m, k), dtype=np.int8)
    rs = np.empty(m, dtype=np.float32)
    lib().orc_quantize_static(_ptr(x), m, k, in_scale, _ptr(q), _ptr(rs))
    return q, rs


def qat_epilogue(acc, rs, ws, out_scale):
    acc = np.ascontiguousarray(acc, dtype=np.int64)
    m, n = acc.shape
    y = np.empty((m, n), dtype=np.float32)
    lib().orc_qat_epilogue(_ptr(acc), _ptr(np.ascontiguousarray(rs, dtype=np.float32)),
                           _ptr(np.ascontiguousarray(ws, dtype=np.float32)), m, n, out_scale, _ptr(y))
    return y


# ------------------------------------------------------- int8 products ----
def matmul_i8_raw(a, w, threads=None):
    a = np.ascontiguousarray(a, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    m, k = a.shape
    n = w.shape[0]
    c = np.empty((m, n), dtype=np.int64)
    lib().orc_matmul_i8_raw(_ptr(a), _ptr(w), m, n, k, _ptr(c), threads or threads_default())
    return c


def i8_block_partials(a, w, threads=None):
    a = np.ascontiguousarray(a, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    m, k = a.shape
    n = w.shape[0]
    p = np.empty((m, n, k // 32), dtype=np.int32)
    lib().orc_i8_block_partials(_ptr(a), _ptr(w), m, n, k, _ptr(p), threads or threads_default())
    return p


def emu_matmul_gw(aq, a_s, a_group, wq, w_s, w_group, threads=None):
    aq = np.ascontiguousarray(aq, dtype=np.int8)
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    a_s = np.ascontiguousarray(a_s, dtype=np.float32)
    w_s = np.ascontiguousarray(w_s, dtype=np.float32)
    m, k = aq.shape
    n = wq.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    lib().orc_emu_matmul_gw(_ptr(aq), _ptr(a_s), a_group, m, k, _ptr(wq), _ptr(w_s), w_group, n, _ptr(out),
                            threads or threads_default())
    return out


# ----------------------------------------------------------- attention ----
def mask_keep(mode, window, t, j):
    return bool(lib().orc_mask_keep(mode, window, t, j))


def _attn(fn, dtype, q, k, v, n_head, n_kv_heads, head_dim, scale, softcap, mode, window, q0, k0, threads):
    q, k, v = _u16(q), _u16(k), _u16(v)
    n_q, n_kv = q.shape[0], k.shape[0]
    assert q.shape == (n_q, n_head * head_dim) and k.shape == (n_kv, n_kv_heads * head_dim) == v.shape
    out = np.empty((n_q, n_head * head_dim), dtype=dtype)
    fn(_ptr(q), _ptr(k), _ptr(v), n_q, n_kv, n_head, n_kv_heads, head_dim, float(scale), float(softcap or 0.0),
       mode, window, q0, k0, _ptr(out), threads or threads_default())
    return out


def attention_ref(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap=0.0, mode=0, window=-1, q0=0, k0=0,
                  threads=None):
    """f64 flash_attn_ref restatement on token-major f16 inputs → f64."""
    return _attn(lib().orc_attention_ref, np.float64, q, k, v, n_head, n_kv_heads, head_dim, scale, softcap,
                 mode, window, q0, k0, threads)


def attention_flex(q, k, v, n_head, n_kv_heads, head_dim, scale, softcap=0.0, mode=0, window=-1, q0=0, k0=0,
                   threads=None):
    """f32 TILE_KV=64 online-softmax restatement of the Burn CPU attention → f32."""
    return _attn(lib().orc_attention_flex, np.float32, q, k, v, n_head, n_kv_heads, head_dim, scale, softcap,
                 mode, window, q0, k0, threads)


# ----------------------------------------------------------------- MoE ----
def route(logits, top_k, norm_topk=True):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    s, e = logits.shape
    ids = np.empty((s, top_k), dtype=np.uint32)
    wts = np.empty((s, top_k), dtype=np.float32)
    lib().orc_route(_ptr(logits), s, e, top_k, int(norm_topk), _ptr(ids), _ptr(wts))
    return ids, wts


def moe_experts(x, ids, wts, gq, gs, uq, us, dq, ds, threads=None, y0=None):
    """W8A8 expert FFN + combine, activations (x and silu·up) quantized per row
    per 32-value group as the reference's expert workers do. gq/uq [E,I,H]
    int8, gs/us [E,I,H/32] f32, dq [E,H,I] int8, ds [E,H,I/32] f32 → y [s,H].
    With y0 (the residual [s,H]) the expert outputs are added onto it in
    ascending expert id, as the reference's layer does (model.rs:606-614)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    s, H = x.shape
    E, I = gq.shape[0], gq.shape[1]
    top_k = ids.shape[1]
    y = np.empty((s, H), dtype=np.float32) if y0 is None else np.array(y0, dtype=np.float32, copy=True)
    arrs = [np.ascontiguousarray(a, dtype=t) for a, t in
            ((ids, np.uint32), (wts, np.float32), (gq, np.int8), (gs, np.float32), (uq, np.int8),
             (us, np.float32), (dq, np.int8), (ds, np.float32))]
    lib().orc_moe_experts(_ptr(x), s, H, I, E, top_k, *[_ptr(a) for a in arrs], _ptr(y),
                          int(y0 is not None), threads or threads_default())
    return y


# ------------------------------------------------------------- metrics ----
def f32_to_bf16(x):
    """f32 → bf16 bits with round-to-nearest-even, NaN kept quiet (the `half`
    crate 2.7.1 bf16::from_f32 behind floats_tensor, ext.rs:1040-1050)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    r = ((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(h):
    """bf16 bits → f32 (exact)."""
    return (np.ascontiguousarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def gelu_tanh(x):
    """orc_gelu_tanh elementwise over f32 (host.rs:12-18)."""
    x = np.ascontiguousarray(x, np.float32)
    f = lib().orc_gelu_tanh
    return np.array([f(float(v)) for v in x.ravel()], np.float32).reshape(x.shape)


def _glue(fn, gate, up):
    g = np.ascontiguousarray(gate, np.float32)
    u = np.ascontiguousarray(up, np.float32)
    assert g.shape == u.shape
    out = np.empty_like(g)
    fn(_ptr(g), _ptr(u), _ptr(out), ctypes.c_int64(g.size))
    return out


def silu_mul(gate, up):
    """silu(gate)·up in f32 (host.rs:30-39)."""
    return _glue(lib().orc_silu_mul, gate, up)


def clef_silu_mul(gate, up):
    """silu(gate)·up with Clef's silu v / (1 + e^-v) in f32, libm expf
    (src/clef/model.rs:491-493): the MoE expert activation."""
    return _glue(lib().orc_clef_silu_mul, gate, up)


def gelu_mul(gate, up):
    """gelu_tanh(gate)·up in f32 (host.rs:20-28)."""
    return _glue(lib().orc_gelu_mul, gate, up)


def rms_norm(x, w, eps):
    """RMSNorm over the last dim in f32 (host.rs:40-56); w None: scale-free."""
    x = np.ascontiguousarray(x, np.float32)
    d = x.shape[-1]
    wp = None
    if w is not None:
        w = np.ascontiguousarray(w, np.float32)
        assert w.shape == (d,)
        wp = _ptr(w)
    out = np.empty_like(x)
    lib().orc_rms_norm(_ptr(x), wp, _ptr(out), _c.c_int64(x.size // d), _c.c_int64(d),
                       _c.c_float(eps))
    return out


def rope(x, cos, sin):
    """Rotate-half RoPE of x [B, S, H, D] with cos/sin [S, D/2] in f32 (host.rs:58-75)."""
    x = np.ascontiguousarray(x, np.float32)
    b, s, h, d = x.shape
    cos = np.ascontiguousarray(cos, np.float32)
    sin = np.ascontiguousarray(sin, np.float32)
    assert d % 2 == 0 and cos.shape == (s, d // 2) and sin.shape == (s, d // 2)
    out = np.empty_like(x)
    lib().orc_rope(_ptr(x), _ptr(cos), _ptr(sin), _ptr(out), b, s, h, d)
    return out


def cosine(a, b):
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0 and nb == 0:
        return 1.0
    return float(a @ b / (na * nb))


def max_rel(got, ref, floor_frac=1e-2):
    """max_i |g - r| / max(|r_i|, floor_frac·max|r|)."""
    g = np.asarray(got, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    floor = floor_frac * max(np.abs(r).max(), 1e-30)
    return float((np.abs(g - r) / np.maximum(np.abs(r), floor)).max())
