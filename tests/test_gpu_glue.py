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
