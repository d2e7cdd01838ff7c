"""GPU parity of the fp16 GEMM (K1) against the oracle, through the C ABI.

Gate (fp16 outputs): cosine >= 0.9999 and max relative error <= 1e-2 with the
floor max_i |g - r| / max(|r_i|, 1e-2·max|r|); integer-valued inputs must match
exactly."""
import sys

import numpy as np
import pytest

from burn_rocket import synth

pytestmark = pytest.mark.gpu
COS_MIN, REL_MAX = 0.9999, 1e-2


def note(msg):
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def run_f16(rk, w_id, a16, n):
    m, k = a16.shape
    da = rk.DeviceBuffer.from_array(a16.view(np.uint16))
    dc = rk.DeviceBuffer(m * n * 2)
    rc = rk.lib().rk_matmul_f16_dev(int(w_id), da.ptr, m, k, dc.ptr, None)
    assert rc == 0, rk.lib().rk_last_error()
    rk.synchronize()
    out = dc.download((m, n), np.uint16).view(np.float16)
    da.free()
    dc.free()
    return out


def check(orc, got, ref):
    g = got.astype(np.float32)
    assert np.isfinite(g).all()
    cos, rel = orc.cosine(g, ref), orc.max_rel(g, ref)
    assert cos >= COS_MIN and rel <= REL_MAX, (cos, rel)
    return cos, rel


def test_gemm_f16_config1_full(rk, orc):
    c = synth.GEMM_F16
    s1, s2 = synth.SEEDS["gemm_f16"]
    note(f"fp16 GEMM {c} seeds {s1},{s2}")
    a = synth.normal_f16(s1, (c["m"], c["k"]))
    b = synth.normal_f16(s2, (c["n"], c["k"]), 0.02)
    wid = rk.pack(b)
    got = run_f16(rk, wid, a, c["n"])
    ref = orc.gemm_f16(a, b)
    check(orc, got, ref)
    ref64 = orc.gemm_f16_f64(a[:64], b)
    check(orc, got[:64], ref64)
    # fp16 rounding of an f32-accumulated result: within 1 ulp of f16(ref)
    r16 = ref.astype(np.float16).astype(np.float32)
    ulp = np.abs(np.spacing(r16.astype(np.float16)).astype(np.float32))
    assert (np.abs(got.astype(np.float32) - r16) <= 2 * ulp + 1e-6).mean() > 0.999


@pytest.mark.parametrize("m,k,n", [(1, 8, 1), (7, 24, 5), (65, 136, 97), (130, 4304, 200), (300, 1152, 3456),
                                   (513, 1024, 3072), (64, 2048, 96), (129, 64, 130)])
def test_gemm_f16_shapes(rk, orc, m, k, n):
    note(f"fp16 GEMM m={m} k={k} n={n}")
    r = np.random.default_rng(m * 1000 + n)
    a = r.standard_normal((m, k)).astype(np.float16)
    b = (r.standard_normal((n, k)) * 0.05).astype(np.float16)
    got = run_f16(rk, rk.pack(b), a, n)
    check(orc, got, orc.gemm_f16(a, b))


@pytest.mark.parametrize("m,k,n", [(96, 64, 80), (256, 1024, 384), (37, 4304, 40)])
def test_gemm_f16_integer_inputs_are_exact(rk, orc, m, k, n):
    note(f"fp16 GEMM exact m={m} k={k} n={n}")
    r = np.random.default_rng(7 + m)
    a = r.integers(-3, 4, (m, k)).astype(np.float16)
    b = r.integers(-3, 4, (n, k)).astype(np.float16)
    got = run_f16(rk, rk.pack(b), a, n).astype(np.float32)
    want = (a.astype(np.int64) @ b.astype(np.int64).T).astype(np.float32)
    assert (got == want.astype(np.float16).astype(np.float32)).all()


def test_vision_layer_gemms_full_size(rk, orc):
    c = synth.VISION
    s = c["s"]
    seeds = synth.SEEDS["vision"]
    x = synth.normal_f16(seeds[0], (s, c["hidden"]))
    shapes = [("qkv", 3 * c["hidden"], c["hidden"]), ("out", c["hidden"], c["hidden"]),
              ("fc1", c["mlp"], c["hidden"]), ("fc2", c["hidden"], c["mlp"])]
    rows = np.r_[0:64, s // 2:s // 2 + 64, s - 64:s]
    for i, (name, n, k) in enumerate(shapes):
        note(f"vision {name} m={s} k={k} n={n}")
        w = synth.normal_f16(seeds[1 + i], (n, k), 0.02)
        a = x if k == c["hidden"] else synth.normal_f16(seeds[5], (s, k))
        got = run_f16(rk, rk.pack(w), a, n)
        check(orc, got[rows], orc.gemm_f16(a[rows], w))


def test_host_matmul_api_f32_in_out(rk, orc):
    note("rk_matmul f16 weight, host f32 in/out")
    r = np.random.default_rng(11)
    x = r.standard_normal((2, 50, 256)).astype(np.float32)
    w = (r.standard_normal((96, 256)) * 0.05).astype(np.float32)
    wid = rk.pack(w)
    y = rk.matmul(x, wid)
    assert y.shape == (2, 50, 96) and y.dtype == np.float32
    ref = orc.gemm_f16(orc.f32_to_f16(x.reshape(100, 256)), orc.f32_to_f16(w))
    check(orc, y.reshape(100, 96), ref)
    # the result is an fp16 value widened to f32 (matmul_f16 reads back fp16)
    assert (y.astype(np.float16).astype(np.float32) == y).all()


def test_pack3_concatenates_along_n(rk):
    note("pack3 segmentation")
    r = np.random.default_rng(12)
    x = r.standard_normal((33, 128)).astype(np.float32)
    parts = [(r.standard_normal((n, 128)) * 0.1).astype(np.float32) for n in (64, 32, 40)]
    y3 = rk.matmul(x, rk.pack3(*parts))
    ys = np.concatenate([rk.matmul(x, rk.pack(p)) for p in parts], axis=1)
    assert (y3 == ys).all()
    y2 = rk.matmul(x, rk.pack2(parts[0], parts[1]))
    assert (y2 == ys[:, :96]).all()


def test_shape_errors_are_reported(rk):
    note("error paths")
    wid = rk.pack(np.ones((16, 64), np.float32))
    with pytest.raises(AssertionError):
        rk.matmul(np.ones((4, 32), np.float32), wid)
    with pytest.raises(rk.RocketError) as e:
        rk.pack(np.ones((16, 12), np.float32))  # K % 8 != 0
    assert e.value.rc == rk.RK_E_SHAPE
    lib = rk.lib()
    # an unknown id is a bad argument (RK_E_RANGE is kept for fp16 range, error.rs:22-24)
    assert lib.rk_matmul(987654321, None, 1, 64, None) == rk.RK_E_SHAPE
    assert b"not packed" in lib.rk_last_error()
    ms = rk.mem_stats()
    assert ms.n_weights >= 1 and ms.weights_bytes >= 16 * 64 * 2


def test_empty_batch_is_a_no_op(rk, orc):
    # The reference's row-chunk loop (ext.rs:1457) runs no chunk for M = 0 and
    # returns an empty [.., 0, N]; every matmul entry returns RK_OK with no
    # launch, while a bad id, K or mode is still reported.
    note("M = 0 on every matmul entry")
    lib = rk.lib()
    k, n = 64, 48
    r = np.random.default_rng(3)
    w = (r.standard_normal((n, k)) * 0.1).astype(np.float32)
    f16, i8 = rk.pack(w), rk.pack_i8(w, 32)
    wq, wd = orc.q8_0_quantize(w)
    q8 = rk.pack_q8_0(orc.q8_0_blocks(wq, wd), n, k)
    f16_glu, q8_glu = rk.pack_f16_glu(w, w), rk.pack_q8_0_glu_f32(w, w)
    for wid in (f16, i8, q8):
        assert rk.matmul(np.zeros((0, k), np.float32), wid).shape == (0, n)
        assert rk.matmul(np.zeros((3, 0, k), np.float32), wid).shape == (3, 0, n)
    calls = [
        ("rk_matmul_f16", lambda kk: lib.rk_matmul_f16(int(f16), None, 0, kk, None)),
        ("rk_matmul_i8_gw", lambda kk: lib.rk_matmul_i8_gw(int(i8), None, None, None, 0, kk, None)),
        ("rk_matmul_i8", lambda kk: lib.rk_matmul_i8(int(i8), None, 0, kk, None)),
        ("rk_matmul_f16_dev", lambda kk: lib.rk_matmul_f16_dev(int(f16), None, 0, kk, None, None)),
        ("rk_matmul_f16_glu_dev",
         lambda kk: lib.rk_matmul_f16_glu_dev(int(f16_glu), None, 0, kk, rk.GLU_SILU, None, 0, None)),
        ("rk_matmul_w8a8_dev", lambda kk: lib.rk_matmul_w8a8_dev(int(q8), None, None, 32, 0, kk, None, None)),
        ("rk_matmul_w8a8_f16out_dev",
         lambda kk: lib.rk_matmul_w8a8_f16out_dev(int(q8), None, None, kk, 0, kk, None, None)),
        ("rk_matmul_w8a8_glu_dev",
         lambda kk: lib.rk_matmul_w8a8_glu_dev(int(q8_glu), None, None, 0, kk, rk.GLU_GELU, None, 1, None)),
        ("rk_matmul_i8_raw_dev", lambda kk: lib.rk_matmul_i8_raw_dev(int(q8), None, 0, kk, None, None)),
        ("rk_matmul_i8_partials_dev", lambda kk: lib.rk_matmul_i8_partials_dev(int(q8), None, 0, kk, None, None)),
        ("rk_quantize_rows_dev", lambda kk: lib.rk_quantize_rows_dev(None, 0, kk, 32, None, None, None)),
    ]
    for name, call in calls:
        assert call(k) == rk.RK_OK, (name, lib.rk_last_error())
        if name != "rk_quantize_rows_dev":
            assert call(k + 32) == rk.RK_E_SHAPE, name  # K still checked
    assert lib.rk_matmul_f16_dev(987654321, None, 0, k, None, None) == rk.RK_E_SHAPE
    assert lib.rk_matmul_f16_glu_dev(int(f16_glu), None, 0, k, 7, None, 0, None) == rk.RK_E_SHAPE
    assert lib.rk_matmul_w8a8_dev(int(q8), None, None, 48, 0, k, None, None) == rk.RK_E_SHAPE
    assert lib.rk_matmul_f16_dev(int(q8), None, 0, k, None, None) == rk.RK_E_UNSUPPORTED
    assert lib.rk_matmul_f16_dev(int(f16), None, -1, k, None, None) == rk.RK_E_SHAPE
    rk.synchronize()


# Every tile configuration of the fp16 kernel (RK_F16_TILE): ragged M and N,
# a K tail inside a 64-value stage, and K of one and two stages (fewer stages
# than the pipeline prologue issues).
F16_TILES = list(range(24))


@pytest.mark.parametrize("tile", F16_TILES)
def test_gemm_f16_every_tile_config(rk, orc, tile, monkeypatch):
    monkeypatch.setenv("RK_F16_TILE", str(tile))
    monkeypatch.setenv("RK_F16_KSPLIT", "1")
    for m, k, n in ((300, 424, 200), (257, 1024, 392), (70, 64, 130), (129, 128, 260)):
        note(f"fp16 GEMM RK_F16_TILE={tile} m={m} k={k} n={n}")
        r = np.random.default_rng(tile * 13 + m + k + n)
        a = r.standard_normal((m, k)).astype(np.float16)
        b = (r.standard_normal((n, k)) * 0.05).astype(np.float16)
        got = run_f16(rk, rk.pack(b), a, n)
        check(orc, got, orc.gemm_f16(a, b))


# Split-K: a tile's K stages over 2, 3 or 4 workgroups whose f32 partials the
# last to arrive sums in split order. Every split of a shape gives the same
# bits from call to call (the order does not depend on which finishes last),
# and the partials' counters are left at zero (a second call is correct).
@pytest.mark.parametrize("tile", [2, 4, 17, 18, 19, 20, 6])
@pytest.mark.parametrize("ksplit", [2, 3, 4])
def test_gemm_f16_split_k(rk, orc, tile, ksplit, monkeypatch):
    monkeypatch.setenv("RK_F16_TILE", str(tile))
    monkeypatch.setenv("RK_F16_KSPLIT", str(ksplit))
    for m, k, n in ((300, 424, 200), (512, 1024, 3072), (70, 256, 130)):
        note(f"fp16 GEMM split-K RK_F16_TILE={tile} ksplit={ksplit} m={m} k={k} n={n}")
        r = np.random.default_rng(tile * 7 + ksplit + m + k + n)
        a = r.standard_normal((m, k)).astype(np.float16)
        b = (r.standard_normal((n, k)) * 0.05).astype(np.float16)
        wid = rk.pack(b)
        got = run_f16(rk, wid, a, n)
        check(orc, got, orc.gemm_f16(a, b))
        again = run_f16(rk, wid, a, n)
        assert (again == got).all()


def test_gemm_f16_split_k_glu(rk, orc, monkeypatch):
    # The gate|up glue epilogue after a split-K sum equals the unsplit launch.
    m, k, n = 300, 512, 200
    r = np.random.default_rng(21)
    x = r.standard_normal((m, k)).astype(np.float16)
    gate = (r.standard_normal((n, k)) * 0.05).astype(np.float32)
    up = (r.standard_normal((n, k)) * 0.05).astype(np.float32)
    wid = rk.pack_f16_glu(gate, up)
    lib = rk.lib()
    da = rk.DeviceBuffer.from_array(x.view(np.uint16))
    outs = []
    for ks in ("1", "3"):
        note(f"fp16 glu GEMM ksplit={ks}")
        monkeypatch.setenv("RK_F16_TILE", "2")
        monkeypatch.setenv("RK_F16_KSPLIT", ks)
        do = rk.DeviceBuffer(m * n * 4)
        assert lib.rk_matmul_f16_glu_dev(int(wid), da.ptr, m, k, rk.GLU_SILU, do.ptr, 0, None) == 0, lib.rk_last_error()
        rk.synchronize()
        outs.append(do.download((m, n), np.float32))
    g = orc.gemm_f16(x, gate.astype(np.float16)).astype(np.float16).astype(np.float32)
    u = orc.gemm_f16(x, up.astype(np.float16)).astype(np.float16).astype(np.float32)
    ref = orc.silu_mul(g, u)
    for got in outs:
        check(orc, got, ref)
