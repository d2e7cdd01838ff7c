"""GPU parity of RMSNorm (weighted and scale-free) and rotate-half RoPE
(ext.rs:75-84, 611-619, 1093-1152; row formulas host.rs:40-75) against the
oracle, through the C ABI.

RoPE evaluates the reference's f32 expressions in the same order without FMA
contraction, so every output type must match the oracle bit for bit.

RMSNorm sums the squares in a fixed parallel order where the reference sums
left to right. The two sums of d non-negative terms differ by at most
(d + d/8 + 6)·2^-24 of the sum (each order's rounding bound, added); the
square root halves that, and the division, square root, reciprocal and the
two products add at most 4 units of 2^-24 of rounding. So f32 outputs obey
|got - ref| <= (0.5·(1.125·d + 6) + 4)·2^-24·|ref|, fp16 / bf16 outputs that
plus one unit in the last place of the 16-bit type, and at least 99 % of the
16-bit outputs must equal the oracle's encoding. Integer-valued rows whose
sum of squares is exact in f32 must match bit for bit in every type."""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
DTS = ("f32", "f16", "bf16")


def note(msg):
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def _code(rk, dt):
    return {"f32": rk.DTYPE_F32, "f16": rk.DTYPE_F16, "bf16": rk.DTYPE_BF16}[dt]


def _encode(orc, x32, dt):
    if dt == "f32":
        return np.ascontiguousarray(x32, np.float32)
    if dt == "f16":
        return np.ascontiguousarray(x32.astype(np.float16))
    return orc.f32_to_bf16(x32)


def _decode(orc, x, dt):
    if dt == "bf16":
        return orc.bf16_to_f32(x)
    return x.astype(np.float32)


def _ulp16(r, dt):
    a = np.maximum(np.abs(r), np.float32(2.0 ** -14 if dt == "f16" else 2.0 ** -126))
    mant = 10 if dt == "f16" else 7
    return np.exp2(np.floor(np.log2(a)) - mant)


class Dev:
    """Device copies of host arrays, each placed `offset` bytes into its buffer."""

    def __init__(self, rk, offset=0):
        self.rk, self.lib, self.offset, self.bufs = rk, rk.lib(), offset, []

    def put(self, a):
        a = np.ascontiguousarray(a)
        buf = self.rk.DeviceBuffer(a.nbytes + self.offset + 16)
        self.bufs.append(buf)
        p = buf.ptr + self.offset
        if a.nbytes:
            self.lib.rk_memcpy_htod(ctypes.c_void_p(p), a.ctypes.data_as(ctypes.c_void_p), a.nbytes)
        return p

    def get(self, p, like):
        self.rk.synchronize()
        out = np.empty_like(like)
        if out.nbytes:
            self.lib.rk_memcpy_dtoh(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(p),
                                    out.nbytes)
        return out

    def free(self):
        for b in self.bufs:
            b.free()


def rms_dev(rk, orc, x32, w32, eps, dt, wdt=None, offset=0, inplace=False):
    wdt = wdt or dt
    x = _encode(orc, x32, dt)
    d = x.shape[-1]
    rows = x.size // d
    dev = Dev(rk, offset)
    try:
        px = dev.put(x)
        po = px if inplace else dev.put(np.zeros_like(x))
        if w32 is None:
            rc = rk.lib().rk_rms_norm_noscale_dev(px, po, rows, d, eps, _code(rk, dt), None)
        else:
            pw = dev.put(_encode(orc, w32, wdt))
            rc = rk.lib().rk_rms_norm_dev(px, pw, _code(rk, wdt), po, rows, d, eps, _code(rk, dt), None)
        assert rc == 0, rk.lib().rk_last_error()
        return _decode(orc, dev.get(po, x), dt), x
    finally:
        dev.free()


def rms_ref(orc, x, w32, eps, dt, wdt=None):
    """The oracle on the values the device saw (inputs decoded from their type)."""
    wdt = wdt or dt
    w = None if w32 is None else _decode(orc, _encode(orc, w32, wdt), wdt)
    return orc.rms_norm(_decode(orc, x, dt), w, eps)


def check_rms(orc, got, ref, d, dt):
    bound = (0.5 * (1.125 * d + 6) + 4) * 2.0 ** -24 * np.abs(ref)
    if dt == "f32":
        assert (np.abs(got - ref) <= bound).all(), np.abs(got - ref).max()
        return
    r16 = _decode(orc, _encode(orc, ref, dt), dt)
    assert (np.abs(got - ref) <= bound + _ulp16(ref, dt)).all()
    assert (got == r16).mean() >= 0.99, (got == r16).mean()


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("rows,d", [(1, 1), (3, 4), (37, 7), (129, 64), (100, 72), (64, 128),
                                    (33, 1152), (17, 2048), (9, 4096), (5, 5000), (3, 8200),
                                    (2, 20000)])
def test_rms_norm_matches_oracle(rk, orc, dt, rows, d):
    note(f"rms_norm {dt} rows={rows} d={d}")
    r = np.random.default_rng(rows * 7919 + d)
    x = (r.standard_normal((rows, d)) * 2).astype(np.float32)
    w = r.standard_normal(d).astype(np.float32)
    got, xe = rms_dev(rk, orc, x, w, 1e-6, dt)
    check_rms(orc, got, rms_ref(orc, xe, w, 1e-6, dt), d, dt)
    got, xe = rms_dev(rk, orc, x, None, 1e-5, dt)
    check_rms(orc, got, rms_ref(orc, xe, None, 1e-5, dt), d, dt)


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("rows,d", [(5, 4), (70, 128), (19, 1152), (4, 4096), (2, 9000)])
def test_rms_norm_exact_sums_are_bit_exact(rk, orc, dt, rows, d):
    note(f"rms_norm exact {dt} rows={rows} d={d}")
    r = np.random.default_rng(d + rows)
    x = r.integers(-8, 9, (rows, d)).astype(np.float32)  # Σx² < 2^24: exact in any order
    w = (r.integers(-64, 65, d) / 16).astype(np.float32)
    for wv in (w, None):
        got, xe = rms_dev(rk, orc, x, wv, 1e-6, dt)
        ref = rms_ref(orc, xe, wv, 1e-6, dt)
        assert (got == _decode(orc, _encode(orc, ref, dt), dt)).all()


def test_rms_norm_mixed_weight_type_misaligned_and_in_place(rk, orc):
    r = np.random.default_rng(5)
    x = r.standard_normal((21, 136)).astype(np.float32)
    w = r.standard_normal(136).astype(np.float32)
    for dt, wdt, off, inplace in (("f16", "f32", 0, False), ("bf16", "f16", 0, True),
                                  ("f16", "f16", 2, False), ("f32", "f32", 4, True),
                                  ("f32", "bf16", 0, False)):
        note(f"rms_norm x {dt} w {wdt} offset {off} in-place {inplace}")
        got, xe = rms_dev(rk, orc, x, w, 1e-6, dt, wdt=wdt, offset=off, inplace=inplace)
        check_rms(orc, got, rms_ref(orc, xe, w, 1e-6, dt, wdt), 136, dt)


def test_rms_norm_zero_rows_and_errors(rk, orc):
    note("rms_norm edge cases")
    lib = rk.lib()
    assert lib.rk_rms_norm_noscale_dev(None, None, 0, 16, 1e-6, rk.DTYPE_F32, None) == 0
    assert lib.rk_rms_norm_noscale_dev(None, None, 4, 0, 1e-6, rk.DTYPE_F32, None) == rk.RK_E_SHAPE
    assert lib.rk_rms_norm_dev(None, None, rk.DTYPE_F32, None, 4, 8, 1e-6, 7, None) == rk.RK_E_SHAPE
    # all-zero rows: out = 0·(eps)^-½ = 0
    got, _ = rms_dev(rk, orc, np.zeros((3, 64), np.float32), np.ones(64, np.float32), 1e-6, "f16")
    assert (got == 0).all()


def test_rms_norm_python_mirror_and_host_form(rk, orc):
    note("rms_norm python mirror, host form")
    r = np.random.default_rng(6)
    x = r.standard_normal((2, 7, 96)).astype(np.float32)
    w = r.standard_normal(96).astype(np.float32)
    ref = orc.rms_norm(x, w, 1e-6)
    check_rms(orc, rk.rms_norm(x, w, 1e-6), ref, 96, "f32")
    check_rms(orc, rk.rms_norm_noscale(x, 1e-6), orc.rms_norm(x, None, 1e-6), 96, "f32")
    y16 = rk.rms_norm(x.astype(np.float16), w.astype(np.float16), 1e-6)
    assert y16.dtype == np.float16 and y16.shape == x.shape
    out = np.empty_like(x)
    lib = rk.lib()
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert lib.rk_rms_norm(p(x), p(w), p(out), 14, 96, 1e-6) == 0
    check_rms(orc, out, ref, 96, "f32")
    assert lib.rk_rms_norm_noscale(p(x), p(out), 14, 96, 1e-6) == 0
    check_rms(orc, out, orc.rms_norm(x, None, 1e-6), 96, "f32")


def rope_dev(rk, orc, x32, c32, s32, dt, cdt=None, offset=0, inplace=False):
    cdt = cdt or dt
    x = _encode(orc, x32, dt)
    c, s = _encode(orc, c32, cdt), _encode(orc, s32, cdt)
    b, sq, h, d = x.shape
    dev = Dev(rk, offset)
    try:
        px, pc, ps = dev.put(x), dev.put(c), dev.put(s)
        po = px if inplace else dev.put(np.zeros_like(x))
        rc = rk.lib().rk_rope_dev(px, pc, ps, _code(rk, cdt), po, b, sq, h, d, _code(rk, dt), None)
        assert rc == 0, rk.lib().rk_last_error()
        got = _decode(orc, dev.get(po, x), dt)
    finally:
        dev.free()
    ref = orc.rope(_decode(orc, x, dt), _decode(orc, c, cdt), _decode(orc, s, cdt))
    return got, _decode(orc, _encode(orc, ref, dt), dt)


def _tables(r, s, half):
    ang = r.uniform(-6, 6, (s, half))
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("shape", [(1, 1, 1, 2), (2, 5, 3, 6), (1, 7, 4, 64), (1, 33, 16, 72),
                                   (2, 40, 8, 128), (1, 3, 2, 4096), (1, 2, 1, 8200)])
def test_rope_bit_exact(rk, orc, dt, shape):
    note(f"rope {dt} shape={shape}")
    r = np.random.default_rng(sum(shape))
    x = r.standard_normal(shape).astype(np.float32)
    c, s = _tables(r, shape[1], shape[3] // 2)
    got, want = rope_dev(rk, orc, x, c, s, dt)
    assert (got == want).all()


@pytest.mark.parametrize("shape,name", [((1, 3633, 16, 128), "Qwen3 q"), ((1, 3633, 8, 128), "Qwen3 k"),
                                        ((1, 2394, 16, 72), "vision")])
def test_rope_full_size(rk, orc, shape, name):
    note(f"rope full size {name} {shape}")
    r = np.random.default_rng(77)
    x = r.standard_normal(shape).astype(np.float32)
    c, s = _tables(r, shape[1], shape[3] // 2)
    got, want = rope_dev(rk, orc, x, c, s, "f16")
    assert (got == want).all()


def test_rope_table_types_misaligned_in_place(rk, orc):
    r = np.random.default_rng(8)
    x = r.standard_normal((2, 9, 3, 40)).astype(np.float32)
    c, s = _tables(r, 9, 20)
    for dt, cdt, off, inplace in (("f16", "f32", 0, False), ("bf16", "f16", 0, True),
                                  ("f16", "f16", 2, False), ("f32", "bf16", 4, True),
                                  ("f32", "f32", 8, False)):
        note(f"rope x {dt} tables {cdt} offset {off} in-place {inplace}")
        got, want = rope_dev(rk, orc, x, c, s, dt, cdt=cdt, offset=off, inplace=inplace)
        assert (got == want).all()


def test_rope_errors_python_mirror_and_host_form(rk, orc):
    note("rope errors, python mirror, host form")
    lib = rk.lib()
    assert lib.rk_rope_dev(None, None, None, rk.DTYPE_F32, None, 1, 2, 3, 5, rk.DTYPE_F32, None) == rk.RK_E_SHAPE
    assert lib.rk_rope_dev(None, None, None, rk.DTYPE_F32, None, 0, 2, 3, 4, rk.DTYPE_F32, None) == 0
    r = np.random.default_rng(9)
    x = r.standard_normal((1, 6, 2, 16)).astype(np.float32)
    c, s = _tables(r, 6, 8)
    want = orc.rope(x, c, s)
    assert (rk.rope_apply(x, c, s) == want).all()
    y = rk.rope_apply(x.astype(np.float16), c.astype(np.float16), s.astype(np.float16))
    assert y.dtype == np.float16
    out = np.empty_like(x)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert lib.rk_rope(p(x), p(c), p(s), p(out), 1, 6, 2, 16) == 0
    assert (out == want).all()


# ---- fused attention prologue on a q|k|v buffer, strided attention ----------
def _qkv_case(r, s, hq, hk, d, pad):
    stride = (hq + 2 * hk) * d + pad
    qkv = r.standard_normal((s, stride)).astype(np.float32)
    wq = (1 + 0.3 * r.standard_normal(d)).astype(np.float32)
    wk = (1 + 0.3 * r.standard_normal(d)).astype(np.float32)
    c, sn = _tables(r, s, d // 2)
    return qkv, stride, wq, wk, c, sn


def qknr_dev(rk, orc, qkv32, stride, hq, hk, d, wq, wk, c32, s32, dt, cdt=None, eps=1e-6):
    cdt = cdt or dt
    x = _encode(orc, qkv32, dt)
    dev = Dev(rk)
    try:
        px = dev.put(x)
        pq = dev.put(_encode(orc, wq, dt)) if wq is not None else None
        pk = dev.put(_encode(orc, wk, dt)) if wk is not None else None
        pc, ps = dev.put(_encode(orc, c32, cdt)), dev.put(_encode(orc, s32, cdt))
        rc = rk.lib().rk_qk_norm_rope_dev(px, x.shape[0], stride, hq, hk, d, pq, pk, eps, pc, ps,
                                          _code(rk, cdt), _code(rk, dt), None)
        assert rc == 0, rk.lib().rk_last_error()
        return _decode(orc, dev.get(px, x), dt), x
    finally:
        dev.free()


def qknr_ref(orc, x, hq, hk, d, wq, wk, c32, s32, dt, cdt=None, eps=1e-6):
    """The reference's composite on the decoded inputs: rms_norm (rounded to the
    element type, as the separate op returns it), then rope, per q and k part."""
    cdt = cdt or dt
    xs = _decode(orc, x, dt)
    s = xs.shape[0]
    cs = _decode(orc, _encode(orc, c32, cdt), cdt)
    sn = _decode(orc, _encode(orc, s32, cdt), cdt)
    out = xs.copy()
    for c0, nh, w in ((0, hq, wq), (hq * d, hk, wk)):
        part = xs[:, c0:c0 + nh * d].reshape(1, s, nh, d)
        if w is not None:
            wv = _decode(orc, _encode(orc, w, dt), dt)
            part = _decode(orc, _encode(orc, orc.rms_norm(part, wv, eps), dt), dt)
        rot = _decode(orc, _encode(orc, orc.rope(part, cs, sn), dt), dt)
        out[:, c0:c0 + nh * d] = rot.reshape(s, nh * d)
    return out


@pytest.mark.parametrize("dt,d", [("f16", 128), ("bf16", 128), ("f32", 128), ("f16", 72),
                                  ("f16", 256), ("f32", 64), ("bf16", 8)])
def test_qk_norm_rope_matches_composite(rk, orc, dt, d):
    hq, hk, s = 4, 2, 77
    note(f"qk_norm_rope {dt} d={d} S={s} {hq}/{hk}")
    r = np.random.default_rng(d * 3 + len(dt))
    qkv, stride, wq, wk, c, sn = _qkv_case(r, s, hq, hk, d, 8)
    got, x = qknr_dev(rk, orc, qkv, stride, hq, hk, d, wq, wk, c, sn, dt)
    want = qknr_ref(orc, x, hq, hk, d, wq, wk, c, sn, dt)
    qk = (hq + hk) * d
    xs = _decode(orc, x, dt)
    assert (got[:, qk:] == xs[:, qk:]).all(), "V columns and row padding must not change"
    g, w = got[:, :qk].reshape(-1, d), want[:, :qk].reshape(-1, d)
    # the norm's f32 result may round to a neighbouring 16-bit value (sum order);
    # RoPE then moves it by at most (|cos| + |sin|) <= 1.5 of that unit
    # (a pair's length is kept, so the row's largest input is at most √2 times
    # its largest output); f32 carries the norm's summation-order bound instead
    wmax = np.abs(w).max(axis=1, keepdims=True)
    if dt == "f32":
        unit = (0.5 * (1.125 * d + 6) + 4) * 2.0 ** -24 * wmax
    else:
        unit = _ulp16(wmax, dt)
        assert (g == w).mean() >= 0.99, (g == w).mean()
    assert (np.abs(g - w) <= 4 * unit).all(), np.abs(g - w).max()


@pytest.mark.parametrize("dt", DTS)
def test_qk_norm_rope_bit_exact_cases(rk, orc, dt):
    hq, hk, s, d = 3, 1, 40, 128
    r = np.random.default_rng(41)
    qkv, stride, wq, wk, c, sn = _qkv_case(r, s, hq, hk, d, 0)
    # integer rows: the sum of squares is exact in any order
    qkv = r.integers(-8, 9, qkv.shape).astype(np.float32)
    wq, wk = (r.integers(-32, 33, d) / 16).astype(np.float32), (r.integers(-32, 33, d) / 16).astype(np.float32)
    note(f"qk_norm_rope exact {dt}")
    got, x = qknr_dev(rk, orc, qkv, stride, hq, hk, d, wq, wk, c, sn, dt)
    assert (got == qknr_ref(orc, x, hq, hk, d, wq, wk, c, sn, dt)).all()
    # no norm weights: RoPE alone, bit-exact; f32 tables with 16-bit values
    note(f"qk_norm_rope rope-only {dt}, f32 tables")
    qkv = r.standard_normal(qkv.shape).astype(np.float32)
    got, x = qknr_dev(rk, orc, qkv, stride, hq, hk, d, None, None, c, sn, dt, cdt="f32")
    assert (got == qknr_ref(orc, x, hq, hk, d, None, None, c, sn, dt, cdt="f32")).all()
    # against the separate device ops (same vector width, so the same sum order)
    note(f"qk_norm_rope vs rk_rms_norm_dev + rk_rope_dev {dt}")
    got, x = qknr_dev(rk, orc, qkv, stride, hq, hk, d, wq, wk, c, sn, dt)
    xs = _decode(orc, x, dt)
    for c0, nh, w in ((0, hq, wq), (hq * d, hk, wk)):
        part = xs[:, c0:c0 + nh * d].reshape(1, s, nh, d)
        normed, _ = rms_dev(rk, orc, part, w, 1e-6, dt)
        rot, _ = rope_dev(rk, orc, normed, c, sn, dt)
        assert (got[:, c0:c0 + nh * d] == rot.reshape(s, nh * d)).all()


def test_qk_norm_rope_errors(rk):
    note("qk_norm_rope errors")
    lib = rk.lib()
    f16 = rk.DTYPE_F16
    buf = rk.DeviceBuffer(4096)
    p = buf.ptr
    assert lib.rk_qk_norm_rope_dev(p, 1, 64, 1, 1, 6, None, None, 1e-6, p, p, f16, f16, None) == 0
    assert lib.rk_qk_norm_rope_dev(p, 1, 64, 1, 1, 7, None, None, 1e-6, p, p, f16, f16, None) == rk.RK_E_SHAPE
    assert lib.rk_qk_norm_rope_dev(p, 1, 8, 1, 1, 8, None, None, 1e-6, p, p, f16, f16, None) == rk.RK_E_SHAPE
    assert lib.rk_qk_norm_rope_dev(p, 1, 64, 1, 1, 8, p, None, 1e-6, p, p, f16, f16, None) == rk.RK_E_SHAPE
    assert lib.rk_qk_norm_rope_dev(p, 1, 64, 1, 1, 8, None, None, 1e-6, p, p, rk.DTYPE_BF16, f16, None) == rk.RK_E_UNSUPPORTED
    # 1024 fp16 values per head: more than 64 lanes × 8 values
    assert lib.rk_qk_norm_rope_dev(p, 0, 2048, 1, 1, 1024, None, None, 1e-6, p, p, f16, f16, None) == 0
    rk.synchronize()
    buf.free()


def _attn_strided(rk, qkv, hq, hk, d, mode, out_stride, n):
    """Attention on one fp16 [n, stride] q|k|v buffer, read in place."""
    lib = rk.lib()
    stride = qkv.shape[1]
    dev = Dev(rk)
    try:
        p = dev.put(qkv)
        out = np.zeros((n, out_stride), np.float16)
        po = dev.put(out)
        rc = lib.rk_attention_strided_dev(p, stride, p + hq * d * 2, stride, p + (hq + hk) * d * 2,
                                          stride, n, n, hq, hk, d, d ** -0.5, 0.0, mode, -1, 0, 0,
                                          po, out_stride, None)
        assert rc == 0, lib.rk_last_error()
        return dev.get(po, out)
    finally:
        dev.free()


def _attn_packed(rk, q, k, v, hq, hk, d, mode, n):
    lib = rk.lib()
    dev = Dev(rk)
    try:
        pq, pk, pv = dev.put(q), dev.put(k), dev.put(v)
        out = np.zeros((n, hq * d), np.float16)
        po = dev.put(out)
        rc = lib.rk_attention_dev(pq, pk, pv, n, n, hq, hk, d, d ** -0.5, 0.0, mode, -1, 0, 0, po, None)
        assert rc == 0, lib.rk_last_error()
        return dev.get(po, out)
    finally:
        dev.free()


@pytest.mark.parametrize("d,hq,hk,mode", [(128, 4, 2, 1), (72, 3, 3, 0), (64, 8, 1, 1)])
def test_attention_strided_on_a_qkv_buffer(rk, d, hq, hk, mode):
    n = 301
    note(f"strided attention d={d} {hq}/{hk} mode={mode} n={n}")
    r = np.random.default_rng(d + hq)
    stride = (hq + 2 * hk) * d + 16
    qkv = r.standard_normal((n, stride)).astype(np.float16)
    q = np.ascontiguousarray(qkv[:, :hq * d])
    k = np.ascontiguousarray(qkv[:, hq * d:(hq + hk) * d])
    v = np.ascontiguousarray(qkv[:, (hq + hk) * d:(hq + 2 * hk) * d])
    want = _attn_packed(rk, q, k, v, hq, hk, d, mode, n)
    out_stride = hq * d + 24
    got = _attn_strided(rk, qkv, hq, hk, d, mode, out_stride, n)
    assert (got[:, :hq * d].view(np.uint16) == want.view(np.uint16)).all()
    assert (got[:, hq * d:] == 0).all()


def test_attention_strided_errors(rk):
    note("strided attention errors")
    lib = rk.lib()
    buf = rk.DeviceBuffer(1 << 16)
    p = buf.ptr
    # stride shorter than the heads; stride not a multiple of 8
    assert lib.rk_attention_strided_dev(p, 64, p, 64, p, 64, 4, 4, 2, 1, 64, 0.1, 0.0, 0, -1, 0, 0, p, 128, None) == rk.RK_E_SHAPE
    assert lib.rk_attention_strided_dev(p, 132, p, 68, p, 68, 4, 4, 2, 1, 64, 0.1, 0.0, 0, -1, 0, 0, p, 128, None) == rk.RK_E_SHAPE
    buf.free()


@pytest.mark.parametrize("groups", ["1", "2", "4"])
def test_qk_norm_rope_row_groups(rk, orc, groups, monkeypatch):
    monkeypatch.setenv("RK_QKNR_GROUPS", groups)
    hq, hk, s, d = 5, 3, 61, 128
    note(f"qk_norm_rope RK_QKNR_GROUPS={groups} S={s} {hq}/{hk}")
    r = np.random.default_rng(43)
    qkv, stride, wq, wk, c, sn = _qkv_case(r, s, hq, hk, d, 8)
    qkv = r.integers(-8, 9, qkv.shape).astype(np.float32)
    got, x = qknr_dev(rk, orc, qkv, stride, hq, hk, d, wq, wk, c, sn, "f16")
    assert (got == qknr_ref(orc, x, hq, hk, d, wq, wk, c, sn, "f16")).all()


def test_qwen3_attention_chain_in_place(rk, orc):
    """qkv GEMM into one buffer → q/k norm + RoPE in place → attention reading q, k, v where
    they lie; against the same ops on separate tensors (bit for bit) and the oracle."""
    s, hid, hq, hk, d = 203, 256, 4, 2, 128
    width = (hq + 2 * hk) * d
    note(f"Qwen3 attention chain S={s} hidden={hid} {hq}/{hk} d={d}")
    r = np.random.default_rng(44)
    x = r.standard_normal((s, hid)).astype(np.float16)
    w = (r.standard_normal((width, hid)) * 0.06).astype(np.float16)
    wq = (1 + 0.2 * r.standard_normal(d)).astype(np.float16)
    wk = (1 + 0.2 * r.standard_normal(d)).astype(np.float16)
    ang = np.arange(s)[:, None] * (10000.0 ** (-np.arange(d // 2) / (d // 2)))[None, :]
    cs, sn = np.cos(ang).astype(np.float16), np.sin(ang).astype(np.float16)
    lib = rk.lib()
    wid = rk.pack(w)
    dev = Dev(rk)
    try:
        px = dev.put(x)
        pqkv = dev.put(np.zeros((s, width), np.float16))
        rc = lib.rk_matmul_f16_dev(int(wid), px, s, hid, pqkv, None)
        assert rc == 0, lib.rk_last_error()
        qkv0 = dev.get(pqkv, np.zeros((s, width), np.float16))  # the projection, before the prologue
        pw, pk, pc, ps = dev.put(wq), dev.put(wk), dev.put(cs), dev.put(sn)
        assert lib.rk_qk_norm_rope_dev(pqkv, s, width, hq, hk, d, pw, pk, 1e-6, pc, ps,
                                       rk.DTYPE_F16, rk.DTYPE_F16, None) == 0, lib.rk_last_error()
        po = dev.put(np.zeros((s, hq * d), np.float16))
        assert lib.rk_attention_strided_dev(pqkv, width, pqkv + hq * d * 2, width, pqkv + (hq + hk) * d * 2,
                                            width, s, s, hq, hk, d, d ** -0.5, 0.0, 1, -1, 0, 0, po,
                                            hq * d, None) == 0, lib.rk_last_error()
        got = dev.get(po, np.zeros((s, hq * d), np.float16))
    finally:
        dev.free()
    # the same steps on separate tensors: sliced q, k, v, the separate norm and RoPE ops,
    # then rk_attention_dev
    q = qkv0[:, :hq * d].astype(np.float32).reshape(1, s, hq, d)
    k = qkv0[:, hq * d:(hq + hk) * d].astype(np.float32).reshape(1, s, hk, d)
    v = qkv0[:, (hq + hk) * d:].copy()
    c32, s32 = cs.astype(np.float32), sn.astype(np.float32)
    qn, _ = rms_dev(rk, orc, q, wq.astype(np.float32), 1e-6, "f16")
    kn, _ = rms_dev(rk, orc, k, wk.astype(np.float32), 1e-6, "f16")
    qr, _ = rope_dev(rk, orc, qn, c32, s32, "f16")
    kr, _ = rope_dev(rk, orc, kn, c32, s32, "f16")
    q16 = qr.reshape(s, hq * d).astype(np.float16)
    k16 = kr.reshape(s, hk * d).astype(np.float16)
    want = _attn_packed(rk, q16, k16, v, hq, hk, d, 1, s)
    assert (got.view(np.uint16) == want.view(np.uint16)).all()
    # and the oracle's f64 attention on those q, k, v (fp16 output gate)
    ref = orc.attention_ref(q16, k16, v, hq, hk, d, d ** -0.5, 0.0, 1)
    g = got.astype(np.float64)
    cos = (g * ref).sum() / np.sqrt((g * g).sum() * (ref * ref).sum())
    assert cos >= 0.9999 and orc.max_rel(g, ref) <= 1e-2


@pytest.mark.parametrize("hq,hk,s", [(2, 0, 9), (0, 3, 9), (1, 1, 1), (7, 1, 2)])
def test_qk_norm_rope_head_counts(rk, orc, hq, hk, s):
    d = 64
    note(f"qk_norm_rope heads {hq}/{hk} S={s}")
    r = np.random.default_rng(hq * 10 + hk + s)
    qkv, stride, wq, wk, c, sn = _qkv_case(r, s, hq, hk, d, 8)
    qkv = r.integers(-8, 9, qkv.shape).astype(np.float32)
    for dt in ("f16", "f32"):
        got, x = qknr_dev(rk, orc, qkv, stride, hq, hk, d, wq, wk, c, sn, dt)
        assert (got == qknr_ref(orc, x, hq, hk, d, wq, wk, c, sn, dt)).all()


@pytest.mark.parametrize("s,hq,hk,d,mode", [(203, 4, 2, 128, 1), (150, 3, 3, 72, 0), (64, 8, 1, 64, 1),
                                            (1, 2, 1, 128, 1), (300, 3, 1, 256, 0), (300, 3, 1, 256, 1)])
def test_attention_qkv_equals_prologue_then_strided_attention(rk, orc, s, hq, hk, d, mode):
    note(f"rk_attention_qkv_dev S={s} {hq}/{hk} d={d} mode={mode}")
    width = (hq + 2 * hk) * d + 8
    r = np.random.default_rng(s + d)
    qkv = (r.standard_normal((s, width)) * 2).astype(np.float16)
    wq = (1 + 0.2 * r.standard_normal(d)).astype(np.float16)
    wk = (1 + 0.2 * r.standard_normal(d)).astype(np.float16)
    ang = np.arange(s)[:, None] * (10000.0 ** (-np.arange(d // 2) / (d // 2)))[None, :]
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    lib = rk.lib()
    outs = []
    for fused in (False, True):
        dev = Dev(rk)
        try:
            p = dev.put(qkv)
            pw, pk, pc, ps = dev.put(wq), dev.put(wk), dev.put(cs), dev.put(sn)
            po = dev.put(np.zeros((s, hq * d), np.float16))
            if fused:
                rc = lib.rk_attention_qkv_dev(p, s, width, hq, hk, d, pw, pk, 1e-6, pc, ps, rk.DTYPE_F32,
                                              d ** -0.5, 0.0, mode, -1, 0, 0, po, hq * d, None)
                assert rc == 0, lib.rk_last_error()
            else:
                assert lib.rk_qk_norm_rope_dev(p, s, width, hq, hk, d, pw, pk, 1e-6, pc, ps, rk.DTYPE_F32,
                                               rk.DTYPE_F16, None) == 0, lib.rk_last_error()
                assert lib.rk_attention_strided_dev(p, width, p + hq * d * 2, width, p + (hq + hk) * d * 2, width,
                                                    s, s, hq, hk, d, d ** -0.5, 0.0, mode, -1, 0, 0, po, hq * d,
                                                    None) == 0, lib.rk_last_error()
            outs.append((dev.get(po, np.zeros((s, hq * d), np.float16)), dev.get(p, qkv)))
        finally:
            dev.free()
    (o0, b0), (o1, b1) = outs
    assert (b0.view(np.uint16) == b1.view(np.uint16)).all(), "the buffer after the prologue"
    assert (o0.view(np.uint16) == o1.view(np.uint16)).all(), "the attention output"


def rms_quant_dev(rk, orc, x32, w32, dt, eps=1e-6):
    x = _encode(orc, x32, dt)
    rows, d = x.shape
    dev = Dev(rk)
    try:
        px = dev.put(x)
        pw = dev.put(_encode(orc, w32, dt)) if w32 is not None else None
        pq = dev.put(np.zeros((rows, d), np.int8))
        ps = dev.put(np.zeros(rows, np.float32))
        rc = rk.lib().rk_rms_norm_quantize_dev(px, pw, _code(rk, dt), rows, d, eps, _code(rk, dt), pq, ps, None)
        assert rc == 0, rk.lib().rk_last_error()
        return dev.get(pq, np.zeros((rows, d), np.int8)), dev.get(ps, np.zeros(rows, np.float32)), x
    finally:
        dev.free()


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("rows,d", [(1, 32), (37, 64), (300, 1024), (9, 2048), (5, 4096)])
def test_rms_norm_quantize_equals_the_two_ops(rk, orc, dt, rows, d):
    if dt == "f32" and d > 2048:
        pytest.skip("f32 rows above 2048 values are outside the fused kernel (RK_E_UNSUPPORTED)")
    note(f"rms_norm_quantize {dt} rows={rows} d={d}")
    r = np.random.default_rng(rows + d)
    x32 = (r.standard_normal((rows, d)) * 3).astype(np.float32)
    w32 = (1 + 0.3 * r.standard_normal(d)).astype(np.float32)
    for w in (w32, None):
        q, sc, x = rms_quant_dev(rk, orc, x32, w, dt)
        # the separate device ops: rk_rms_norm_dev in dt, then rk_quantize_rows_dev per token
        y, _ = rms_dev(rk, orc, _decode(orc, x, dt), w, 1e-6, dt)
        dev = Dev(rk)
        try:
            py = dev.put(y.astype(np.float32))
            pq, ps = dev.put(np.zeros((rows, d), np.int8)), dev.put(np.zeros(rows, np.float32))
            assert rk.lib().rk_quantize_rows_dev(py, rows, d, d, pq, ps, None) == 0
            q2, s2 = dev.get(pq, q), dev.get(ps, sc)
        finally:
            dev.free()
        assert (q == q2).all() and (sc.view(np.uint32) == s2.view(np.uint32)).all()


@pytest.mark.parametrize("dt", DTS)
def test_rms_norm_quantize_exact_rows_match_the_oracle(rk, orc, dt):
    rows, d = 70, 512
    note(f"rms_norm_quantize vs oracle, integer rows, {dt}")
    r = np.random.default_rng(9)
    x32 = r.integers(-8, 9, (rows, d)).astype(np.float32)
    w32 = (r.integers(-32, 33, d) / 16).astype(np.float32)
    q, sc, x = rms_quant_dev(rk, orc, x32, w32, dt)
    y = _decode(orc, _encode(orc, orc.rms_norm(_decode(orc, x, dt), _decode(orc, _encode(orc, w32, dt), dt), 1e-6), dt), dt)
    qo, so = orc.quantize_rows(y, d)
    assert (q == qo).all() and (sc == so[:, 0]).all()


def test_rms_norm_quantize_rejects_what_it_does_not_fuse(rk):
    note("rms_norm_quantize errors")
    lib = rk.lib()
    buf = rk.DeviceBuffer(1 << 16)
    p = buf.ptr
    f16 = rk.DTYPE_F16
    assert lib.rk_rms_norm_quantize_dev(p, None, f16, 4, 12, 1e-6, f16, p, p, None) == rk.RK_E_UNSUPPORTED
    assert lib.rk_rms_norm_quantize_dev(p, p, rk.DTYPE_F32, 4, 64, 1e-6, f16, p, p, None) == rk.RK_E_UNSUPPORTED
    assert lib.rk_rms_norm_quantize_dev(p, None, f16, 2, 8192, 1e-6, f16, p, p, None) == rk.RK_E_UNSUPPORTED
    assert lib.rk_rms_norm_quantize_dev(p, None, f16, 0, 64, 1e-6, f16, p, p, None) == 0
    buf.free()
