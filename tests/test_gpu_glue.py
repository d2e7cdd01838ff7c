"""GPU parity of the MLP glue ops (silu·up, gelu·up; ext.rs:603-608,
1057-1090, formulas host.rs:12-39) against the oracle, through the C ABI.

The device evaluates the reference's f32 formula in the same order without
FMA contraction, but its exp and tanh are the device library's, an ulp or so
from the host libm the oracle calls. gelu's tanh(·)+1 cancels for negative
gates and scales that difference by |gate·up|, so the bound is
|got - ref| <= 4e-6·|ref| + 2^-22·|gate·up| (+ half a unit in the last place
of fp16 / bf16 outputs, which are rounded to nearest even); at least 99 % of
the 16-bit outputs must equal the oracle's encoding, which pins the rounding.
Values compare as numbers: where the host's tanh reaches -1 exactly the
reference yields -0.0 and the device may yield +0.0."""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
OPS = {"silu": ("rk_silu_mul_dev", "silu_mul"), "gelu": ("rk_gelu_mul_dev", "gelu_mul")}


def note(msg):
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def _encode(x32, dt):
    if dt == "f32":
        return x32.astype(np.float32)
    if dt == "f16":
        return x32.astype(np.float16)
    import oracle as orc
    return orc.f32_to_bf16(x32)


def _decode(x, dt):
    if dt == "bf16":
        import oracle as orc
        return orc.bf16_to_f32(x)
    return x.astype(np.float32)


def _run(rk, op, a, b, dt, offset=0, inplace=False):
    """Device op on copies of a, b placed `offset` elements into fresh buffers."""
    code = {"f32": rk.DTYPE_F32, "f16": rk.DTYPE_F16, "bf16": rk.DTYPE_BF16}[dt]
    es = a.itemsize
    n = a.size
    bufs = [rk.DeviceBuffer((n + offset) * es + 16) for _ in range(3)]
    pa, pb, po = (buf.ptr + offset * es for buf in bufs)
    lib = rk.lib()
    lib.rk_memcpy_htod(ctypes.c_void_p(pa), a.ctypes.data_as(ctypes.c_void_p), a.nbytes)
    lib.rk_memcpy_htod(ctypes.c_void_p(pb), b.ctypes.data_as(ctypes.c_void_p), b.nbytes)
    out_ptr = pa if inplace else po
    rc = getattr(lib, OPS[op][0])(pa, pb, out_ptr, n, code, None)
    assert rc == 0, lib.rk_last_error()
    rk.synchronize()
    got = np.empty_like(a)
    lib.rk_memcpy_dtoh(got.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(out_ptr), a.nbytes)
    for buf in bufs:
        buf.free()
    return got


def _expect(orc, op, a, b, dt):
    ref32 = getattr(orc, OPS[op][1])(_decode(a, dt), _decode(b, dt))
    return ref32, _encode(ref32, dt)


def _check(got, ref32, ref_enc, dt, g32, u32):
    gv = _decode(got, dt) if dt != "f32" else got
    half_ulp = {"f32": 0.0, "f16": 2.0 ** -11, "bf16": 2.0 ** -8}[dt]
    floor = {"f32": 0.0, "f16": 2.0 ** -25, "bf16": 0.0}[dt]
    bound = (4e-6 + half_ulp) * np.abs(ref32) + 2.0 ** -22 * np.abs(g32 * u32) + floor
    err = np.abs(gv.astype(np.float64) - ref32)
    assert (err <= bound).all(), (err - bound).max()
    if dt != "f32":
        same = (gv == _decode(ref_enc, dt))  # as values: +0 == -0
        assert same.mean() >= 0.99, same.mean()


@pytest.mark.parametrize("op", ["silu", "gelu"])
@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("n,offset", [(1, 0), (7, 0), (4096 + 3, 0), (1 << 18, 0), (1001, 1), (4099, 3)])
def test_glue_against_oracle(rk, orc, op, dt, n, offset):
    note(f"glue {op} {dt} n={n} offset={offset}")
    r = np.random.default_rng(n + offset + len(op) * 7 + len(dt))
    a32 = (r.standard_normal(n) * 4).astype(np.float32)
    b32 = r.standard_normal(n).astype(np.float32)
    a, b = _encode(a32, dt), _encode(b32, dt)
    got = _run(rk, op, a, b, dt, offset)
    _check(got, *_expect(orc, op, a, b, dt), dt, _decode(a, dt), _decode(b, dt))


@pytest.mark.parametrize("op", ["silu", "gelu"])
def test_glue_in_place_and_reference_vectors(rk, orc, op):
    note(f"glue {op} in place, host.rs vectors")
    gate = np.array([0.0, 1.0, -1.0, 3.7, -12.5], np.float32)
    up = np.array([2.0, -1.0, 0.5, 0.25, 8.0], np.float32)
    got = _run(rk, op, gate, up, "f32", inplace=True)
    _check(got, *_expect(orc, op, gate, up, "f32"), "f32", gate, up)
    # the Python mirror and the host-buffer entry point
    fn = getattr(rk, OPS[op][1])
    assert (fn(gate, up) == got).all()
    host = np.empty_like(gate)
    name = "rk_silu_mul" if op == "silu" else "rk_gelu_mul"
    assert getattr(rk.lib(), name)(gate.ctypes.data, up.ctypes.data, host.ctypes.data, 5) == 0
    assert (host == got).all()
    assert fn(np.zeros((0,), np.float16), np.zeros((0,), np.float16)).shape == (0,)


def test_glue_errors(rk):
    note("glue error paths")
    lib = rk.lib()
    assert lib.rk_silu_mul_dev(None, None, None, 4, 0, None) == rk.RK_E_SHAPE
    assert lib.rk_gelu_mul_dev(None, None, None, 0, 7, None) == rk.RK_E_SHAPE
    assert lib.rk_silu_mul_dev(None, None, None, 0, 0, None) == 0
    with pytest.raises(AssertionError):
        rk.silu_mul(np.ones(3, np.float32), np.ones(3, np.float16))
    with pytest.raises(AssertionError):
        rk.gelu_mul(np.ones(3, np.float32), np.ones(4, np.float32))


# fp16 gate|up GEMM with the glue in its epilogue (the reference's Qwen3 MLP:
# one fp16 matmul on pack2(gate, up), slice, silu_mul; src/qwen3_embedding/
# model.rs:592-600). Against the oracle: the two fp16 products rounded to fp16,
# then its glue; against the unfused GPU path (two fp16 GEMMs, then the glue op
# on their f32-widened outputs): bit for bit, since each output element sees
# the same f32 accumulation, the same fp16 rounding and the same glue formula.
@pytest.mark.parametrize("glu", ["silu", "gelu"])
@pytest.mark.parametrize("m,k,n", [(3633, 1024, 3072), (100, 256, 72), (257, 512, 200)])
def test_f16_glu_gemm(rk, orc, m, k, n, glu):
    note(f"fp16 gate|up GEMM + {glu}: m={m} k={k} n={n}")
    lib = rk.lib()
    r = np.random.default_rng(m + n + (glu == "gelu"))
    x = r.standard_normal((m, k)).astype(np.float16)
    gate = (r.standard_normal((n, k)) * 0.05).astype(np.float32)
    up = (r.standard_normal((n, k)) * 0.05).astype(np.float32)
    code = rk.GLU_SILU if glu == "silu" else rk.GLU_GELU
    wid = rk.pack_f16_glu(gate, up)
    dx = rk.DeviceBuffer.from_array(x.view(np.uint16))
    outs = {}
    for f16out in (0, 1):
        do = rk.DeviceBuffer(m * n * (2 if f16out else 4))
        assert lib.rk_matmul_f16_glu_dev(int(wid), dx.ptr, m, k, code, do.ptr, f16out, None) == 0, \
            lib.rk_last_error()
        rk.synchronize()
        outs[f16out] = (do.download((m, n), np.uint16).view(np.float16).astype(np.float32) if f16out
                        else do.download((m, n), np.float32))
    # oracle: fp16 products (f32 accumulation, rounded to fp16), then the glue
    g16 = orc.f16_to_f32(orc.f32_to_f16(orc.gemm_f16(x, orc.f32_to_f16(gate))))
    u16 = orc.f16_to_f32(orc.f32_to_f16(orc.gemm_f16(x, orc.f32_to_f16(up))))
    ref = orc.silu_mul(g16, u16) if glu == "silu" else orc.gelu_mul(g16, u16)
    for f16out, got in outs.items():
        cos, rel = orc.cosine(got, ref), orc.max_rel(got, ref)
        assert cos >= 0.9999 and rel <= 1e-2, (f16out, cos, rel)
    # unfused GPU path on the same data
    prods = []
    for w in (gate, up):
        wq = rk.pack(w)
        dc = rk.DeviceBuffer(m * n * 2)
        assert lib.rk_matmul_f16_dev(int(wq), dx.ptr, m, k, dc.ptr, None) == 0
        rk.synchronize()
        prods.append(dc.download((m, n), np.uint16).view(np.float16).astype(np.float32))
    fn = rk.silu_mul if glu == "silu" else rk.gelu_mul
    assert (outs[0] == fn(prods[0], prods[1])).all()
    assert (outs[1] == fn(prods[0].astype(np.float16), prods[1].astype(np.float16)).astype(np.float32)).all()
    # the interleaved weight is refused by the plain fp16 GEMM
    assert lib.rk_matmul_f16_dev(int(wid), dx.ptr, m, k, rk.DeviceBuffer(m * 2 * n * 2).ptr, None) == rk.RK_E_UNSUPPORTED


# Every tile configuration the fp16 GLU epilogue runs on (RK_F16_TILE; gate and
# up tiles pair inside one wave, so the wave tile is a multiple of 32 columns):
# ragged M and N, a K tail, equal bit for bit to the unfused products and glue.
@pytest.mark.parametrize("tile", [0, 1, 2, 3, 4, 8, 22])
def test_f16_glu_gemm_every_tile(rk, orc, tile, monkeypatch):
    lib = rk.lib()
    for m, k, n in ((300, 520, 200), (257, 192, 100)):
        note(f"fp16 gate|up GEMM + silu RK_F16_TILE={tile} m={m} k={k} n={n}")
        r = np.random.default_rng(tile * 31 + m + n)
        x = r.standard_normal((m, k)).astype(np.float16)
        gate = (r.standard_normal((n, k)) * 0.05).astype(np.float32)
        up = (r.standard_normal((n, k)) * 0.05).astype(np.float32)
        wid = rk.pack_f16_glu(gate, up)
        dx = rk.DeviceBuffer.from_array(x.view(np.uint16))
        do = rk.DeviceBuffer(m * n * 4)
        monkeypatch.setenv("RK_F16_TILE", str(tile))
        assert lib.rk_matmul_f16_glu_dev(int(wid), dx.ptr, m, k, rk.GLU_SILU, do.ptr, 0, None) == 0, \
            lib.rk_last_error()
        rk.synchronize()
        got = do.download((m, n), np.float32)
        monkeypatch.delenv("RK_F16_TILE")
        prods = []
        for w in (gate, up):
            dc = rk.DeviceBuffer(m * n * 2)
            assert lib.rk_matmul_f16_dev(int(rk.pack(w)), dx.ptr, m, k, dc.ptr, None) == 0
            rk.synchronize()
            prods.append(dc.download((m, n), np.uint16).view(np.float16).astype(np.float32))
        assert (got == rk.silu_mul(prods[0], prods[1])).all()
        g16 = orc.f16_to_f32(orc.f32_to_f16(orc.gemm_f16(x, orc.f32_to_f16(gate))))
        u16 = orc.f16_to_f32(orc.f32_to_f16(orc.gemm_f16(x, orc.f32_to_f16(up))))
        ref = orc.silu_mul(g16, u16)
        assert orc.cosine(got, ref) >= 0.9999 and orc.max_rel(got, ref) <= 1e-2


def test_cast_dev_every_type_pair_rounds_to_nearest_even(rk, orc):
    # rk_cast_dev: the f32 <-> f16 / bf16 conversions either side of every op
    # (ext.rs:2144-2170), bit for bit against the oracle's RNE conversions
    # (`half` 2.7.1), including ties, subnormals, overflow and ±0.
    note("rk_cast_dev")
    lib = rk.lib()
    r = np.random.default_rng(77)
    x = np.concatenate([r.standard_normal(100001).astype(np.float32) * 10.0 ** r.integers(-8, 6, 100001),
                        np.array([0.0, -0.0, 65504.0, 65520.0, 1e30, -1e30, 5.96e-8, 2.98e-8, 1e-40],
                                 np.float32)]).astype(np.float32)
    as_f32 = {rk.DTYPE_F32: x, rk.DTYPE_F16: orc.f16_to_f32(orc.f32_to_f16(x)),
              rk.DTYPE_BF16: orc.bf16_to_f32(orc.f32_to_bf16(x))}
    bits = {rk.DTYPE_F32: lambda v: v.view(np.uint32), rk.DTYPE_F16: orc.f32_to_f16, rk.DTYPE_BF16: orc.f32_to_bf16}
    size = {rk.DTYPE_F32: 4, rk.DTYPE_F16: 2, rk.DTYPE_BF16: 2}
    for src in (rk.DTYPE_F32, rk.DTYPE_F16, rk.DTYPE_BF16):
        src_bits = bits[src](as_f32[src])
        dx = rk.DeviceBuffer.from_array(src_bits)
        for dst in (rk.DTYPE_F32, rk.DTYPE_F16, rk.DTYPE_BF16):
            dy = rk.DeviceBuffer(x.size * size[dst])
            assert lib.rk_cast_dev(dx.ptr, src, dy.ptr, dst, x.size, None) == 0, lib.rk_last_error()
            rk.synchronize()
            got = dy.download(x.size, np.uint32 if dst == rk.DTYPE_F32 else np.uint16)
            want = bits[dst](as_f32[src])  # the source value is exact in f32
            nan = np.isnan(as_f32[src])
            assert (got[~nan] == want[~nan]).all(), (src, dst)
