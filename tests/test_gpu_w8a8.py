"""GPU parity of the W8A8 / Q8_0 GEMM (K2) against the oracle, through the C ABI.

Integer work is bit-exact: the activation quantizer's codes and scales, the raw
int32 product over the full K and the per-32-block int32 partials. Scaled f32
outputs follow the reference formula up to f32 rounding order and are held to
cosine >= 0.9999, max relative error <= 1e-2 (the fp16-output gate)."""
import sys

import numpy as np
import pytest

from burn_rocket import synth

pytestmark = pytest.mark.gpu
COS_MIN, REL_MAX = 0.9999, 1e-2


def note(msg):
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def _lib(rk):
    return rk.lib()


def dev(rk, a):
    return rk.DeviceBuffer.from_array(a)


def quantize_dev(rk, x, group):
    m, k = x.shape
    dx = dev(rk, x)
    dq = rk.DeviceBuffer(m * k)
    ds = rk.DeviceBuffer(m * (k // group) * 4)
    rc = _lib(rk).rk_quantize_rows_dev(dx.ptr, m, k, group, dq.ptr, ds.ptr, None)
    assert rc == 0, _lib(rk).rk_last_error()
    rk.synchronize()
    return dq, ds


def raw_dev(rk, wid, aq):
    m, k = aq.shape
    n = rk.weight_info(wid)[1]
    da = dev(rk, aq)
    dc = rk.DeviceBuffer(m * n * 4)
    assert _lib(rk).rk_matmul_i8_raw_dev(int(wid), da.ptr, m, k, dc.ptr, None) == 0, _lib(rk).rk_last_error()
    rk.synchronize()
    return dc.download((m, n), np.int32)


def w8a8_dev(rk, wid, dq, ds, a_group, m, k, f16out=False):
    n = rk.weight_info(wid)[1]
    dc = rk.DeviceBuffer(m * n * (2 if f16out else 4))
    fn = _lib(rk).rk_matmul_w8a8_f16out_dev if f16out else _lib(rk).rk_matmul_w8a8_dev
    assert fn(int(wid), dq.ptr, ds.ptr, a_group, m, k, dc.ptr, None) == 0, _lib(rk).rk_last_error()
    rk.synchronize()
    if f16out:
        return dc.download((m, n), np.uint16).view(np.float16).astype(np.float32)
    return dc.download((m, n), np.float32)


def check(orc, got, ref):
    assert np.isfinite(got).all()
    cos, rel = orc.cosine(got, ref), orc.max_rel(got, ref)
    assert cos >= COS_MIN and rel <= REL_MAX, (cos, rel)


@pytest.fixture(scope="module")
def config2(rk, orc):
    c = synth.W8A8
    s1, s2, s3 = synth.SEEDS["w8a8"]
    x_up = synth.normal_f32(s1, (c["m"], c["hidden"]))
    x_dn = synth.normal_f32(s1 + 1000, (c["m"], c["inter"]))
    w_up = synth.normal_f32(s2, (c["inter"], c["hidden"]), 0.02)
    w_dn = synth.normal_f32(s3, (c["hidden"], c["inter"]), 0.02)
    out = {}
    for name, x, w in (("up", x_up, w_up), ("down", x_dn, w_dn)):
        wq, wd = orc.q8_0_quantize(w)
        blocks = orc.q8_0_blocks(wq, wd)
        wid = rk.pack_q8_0(blocks, *w.shape)
        out[name] = dict(x=x, wq=wq, ws=wd.view(np.float16).astype(np.float32), wid=wid)
    return out


def test_activation_quantizer_is_bit_exact(rk, orc, config2):
    for name in ("up", "down"):
        x = config2[name]["x"]
        m, k = x.shape
        for group in (k, 32, 128):
            note(f"quantize_rows {name} m={m} k={k} group={group}")
            dq, ds = quantize_dev(rk, x, group)
            q, s = orc.quantize_rows(x, group)
            assert (dq.download((m, k), np.int8) == q).all()
            assert (ds.download((m, k // group), np.float32).view(np.uint32) == s.view(np.uint32)).all()


def test_raw_int32_full_config2_is_bit_exact(rk, orc, config2):
    for name in ("up", "down"):
        d = config2[name]
        m, k = d["x"].shape
        note(f"raw int32 {name} m={m} k={k} n={d['wq'].shape[0]}")
        aq, _ = orc.quantize_rows(d["x"], k)
        got = raw_dev(rk, d["wid"], aq)
        want = orc.matmul_i8_raw(aq, d["wq"])
        assert (got.astype(np.int64) == want).all()


def test_block_partials_are_bit_exact(rk, orc, config2):
    d = config2["down"]
    rows = 192
    aq, _ = orc.quantize_rows(d["x"][:rows], d["x"].shape[1])
    m, k = aq.shape
    n = d["wq"].shape[0]
    note(f"int32 block partials m={m} k={k} n={n}")
    da = dev(rk, aq)
    dp = rk.DeviceBuffer(m * n * (k // 32) * 4)
    assert _lib(rk).rk_matmul_i8_partials_dev(int(d["wid"]), da.ptr, m, k, dp.ptr, None) == 0
    rk.synchronize()
    got = dp.download((m, n, k // 32), np.int32)
    assert (got == orc.i8_block_partials(aq, d["wq"])).all()


@pytest.mark.parametrize("f16out", [False, True])
def test_per_token_w8a8_full_config2(rk, orc, config2, f16out):
    for name in ("up", "down"):
        d = config2[name]
        m, k = d["x"].shape
        note(f"W8A8 per-token {name} m={m} k={k} f16out={f16out}")
        dq, ds = quantize_dev(rk, d["x"], k)
        got = w8a8_dev(rk, d["wid"], dq, ds, k, m, k, f16out)
        aq, a_s = orc.quantize_rows(d["x"], k)
        ref = orc.emu_matmul_gw(aq, a_s, k, d["wq"], d["ws"], 32)
        check(orc, got, ref)
        if not f16out:
            # only f32 rounding order differs from the reference formula
            assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("f16out", [False, True])
def test_group32_w8a8_full_config2(rk, orc, config2, f16out):
    # The reference's own W8A8 form at config 2: activations quantized per row
    # per 32-value group (quantize_i8_rows, ext.rs:1505-1554), Σ_g (a_s·w_s)·P_g.
    for name in ("up", "down"):
        d = config2[name]
        m, k = d["x"].shape
        note(f"W8A8 group-32 {name} m={m} k={k} f16out={f16out}")
        dq, ds = quantize_dev(rk, d["x"], 32)
        got = w8a8_dev(rk, d["wid"], dq, ds, 32, m, k, f16out)
        aq, a_s = orc.quantize_rows(d["x"], 32)
        ref = orc.emu_matmul_gw(aq, a_s, 32, d["wq"], d["ws"], 32)
        check(orc, got, ref)
        if not f16out:
            assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


# Every tile configuration of the group-32 pipelined path (RK_Q8G_TILE), with
# ragged M and N, odd and even block counts and a K tail inside a stage.
@pytest.mark.parametrize("tile", [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10])
def test_group32_w8a8_every_tile_config(rk, orc, tile, monkeypatch):
    monkeypatch.setenv("RK_Q8G_TILE", str(tile))
    for m, k, n in ((300, 416, 200), (257, 1024, 392), (1, 32, 1)):
        note(f"W8A8 group-32 RK_Q8G_TILE={tile} m={m} k={k} n={n}")
        r = np.random.default_rng(tile * 5 + m + k + n)
        x = r.standard_normal((m, k)).astype(np.float32)
        w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
        wq, wd = orc.q8_0_quantize(w)
        wid = rk.pack_q8_0(orc.q8_0_blocks(wq, wd), n, k)
        aq, a_s = orc.quantize_rows(x, 32)
        dq, ds = quantize_dev(rk, x, 32)
        ref = orc.emu_matmul_gw(aq, a_s, 32, wq, wd.view(np.float16).astype(np.float32), 32)
        for f16out in (False, True):
            got = w8a8_dev(rk, wid, dq, ds, 32, m, k, f16out)
            check(orc, got, ref)
            if not f16out:
                assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("group", [32, 64, 128])
def test_group_wise_host_matmul_matches_matmul_gw(rk, orc, group):
    note(f"rk_matmul pack_i8 group={group}")
    r = np.random.default_rng(group)
    m, k, n = 77, 512, 160
    x = r.standard_normal((m, k)).astype(np.float32)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    wid = rk.pack_i8(w, group)
    y = rk.matmul(x, wid)
    wq, ws = orc.quantize_rows(w, group)
    aq, a_s = orc.quantize_rows(x, group)
    ref = orc.emu_matmul_gw(aq, a_s, group, wq, ws, group)
    check(orc, y, ref)
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    # the resident codes are the oracle's codes: the raw product is exact
    assert (raw_dev(rk, wid, aq).astype(np.int64) == orc.matmul_i8_raw(aq, wq)).all()


@pytest.mark.parametrize("m,k,n", [(1, 32, 1), (5, 160, 40), (130, 4096, 96), (64, 96, 33)])
def test_w8a8_edge_shapes(rk, orc, m, k, n):
    note(f"W8A8 edge m={m} k={k} n={n}")
    r = np.random.default_rng(m + k + n)
    x = r.standard_normal((m, k)).astype(np.float32)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    wq, wd = orc.q8_0_quantize(w)
    wid = rk.pack_q8_0(orc.q8_0_blocks(wq, wd), n, k)
    aq, a_s = orc.quantize_rows(x, k)
    assert (raw_dev(rk, wid, aq).astype(np.int64) == orc.matmul_i8_raw(aq, wq)).all()
    dq, ds = quantize_dev(rk, x, k)
    got = w8a8_dev(rk, wid, dq, ds, k, m, k)
    ref = orc.emu_matmul_gw(aq, a_s, k, wq, wd.view(np.float16).astype(np.float32), 32)
    check(orc, got, ref)


# Every tile configuration of the per-token Q8_0 kernel (RK_Q8_TILE): ragged
# M and N against every tile size, an odd and an even number of 32-value
# blocks (the pipeline alternates register sets per block) and a K tail that
# ends inside a 128-value stage.
Q8_TILES = list(range(24))


@pytest.mark.parametrize("tile", Q8_TILES)
def test_w8a8_every_tile_config(rk, orc, tile, monkeypatch):
    monkeypatch.setenv("RK_Q8_TILE", str(tile))
    for m, k, n in ((300, 416, 200), (257, 1024, 392)):
        note(f"W8A8 RK_Q8_TILE={tile} m={m} k={k} n={n}")
        r = np.random.default_rng(tile * 7 + m + k + n)
        x = r.standard_normal((m, k)).astype(np.float32)
        w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
        wq, wd = orc.q8_0_quantize(w)
        wid = rk.pack_q8_0(orc.q8_0_blocks(wq, wd), n, k)
        aq, a_s = orc.quantize_rows(x, k)
        dq, ds = quantize_dev(rk, x, k)
        ref = orc.emu_matmul_gw(aq, a_s, k, wq, wd.view(np.float16).astype(np.float32), 32)
        for f16out in (False, True):
            got = w8a8_dev(rk, wid, dq, ds, k, m, k, f16out)
            check(orc, got, ref)
            if not f16out:
                assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


# Two K-groups per workgroup (RK_Q8_TILE 24-27; K % 256 == 0): each group
# folds half of K in its own LDS ring and the halves meet in LDS. Ragged M and
# N, K of two, four and twelve 128-value stages per group; the raw int32 form
# (RK_Q8_RAW_TILE=1) stays bit-exact.
@pytest.mark.parametrize("tile", [24, 25, 26, 27])
def test_w8a8_k_groups(rk, orc, tile, monkeypatch):
    monkeypatch.setenv("RK_Q8_TILE", str(tile))
    monkeypatch.setenv("RK_Q8_RAW_TILE", "1")
    for m, k, n in ((300, 512, 200), (257, 1024, 392), (70, 3072, 130)):
        note(f"W8A8 K-groups RK_Q8_TILE={tile} m={m} k={k} n={n}")
        r = np.random.default_rng(tile * 11 + m + k + n)
        x = r.standard_normal((m, k)).astype(np.float32)
        w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
        wq, wd = orc.q8_0_quantize(w)
        wid = rk.pack_q8_0(orc.q8_0_blocks(wq, wd), n, k)
        aq, a_s = orc.quantize_rows(x, k)
        dq, ds = quantize_dev(rk, x, k)
        ref = orc.emu_matmul_gw(aq, a_s, k, wq, wd.view(np.float16).astype(np.float32), 32)
        for f16out in (False, True):
            got = w8a8_dev(rk, wid, dq, ds, k, m, k, f16out)
            check(orc, got, ref)
            if not f16out:
                assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
                again = w8a8_dev(rk, wid, dq, ds, k, m, k, f16out)
                assert (again == got).all()
        assert (raw_dev(rk, wid, aq).astype(np.int64) == orc.matmul_i8_raw(aq, wq)).all()


@pytest.mark.parametrize("in_scale,out_scale", [(0.02, 0.0), (0.0, 0.0), (0.02, 0.05)])
def test_qat_matmul_is_bit_exact(rk, orc, in_scale, out_scale):
    note(f"QAT in_scale={in_scale} out_scale={out_scale}")
    r = np.random.default_rng(5)
    m, k, n = 45, 256, 64
    x = r.standard_normal((m, k)).astype(np.float32)
    codes = r.integers(-127, 128, (n, k), dtype=np.int8)
    ws = (r.uniform(0.5, 1.5, n) * 1e-3).astype(np.float32)
    wid = rk.pack_qat(codes, ws, n, k, in_scale, out_scale)
    y = rk.matmul(x, wid)
    q, rs = orc.quantize_static(x, in_scale)
    ref = orc.qat_epilogue(orc.matmul_i8_raw(q, codes), rs, ws, out_scale)
    assert (y.view(np.uint32) == ref.view(np.uint32)).all()


def test_rewrite_replaces_the_resident_codes(rk, orc):
    note("rewrite_i8")
    r = np.random.default_rng(9)
    m, k, n = 16, 128, 64
    w1 = r.integers(-127, 128, (n, k), dtype=np.int8)
    w2 = r.integers(-127, 128, (n, k), dtype=np.int8)
    s = np.ones((n, k // 32), np.float32)
    wid = rk.pack_i8_codes(w1, s, 32)
    aq = r.integers(-127, 128, (m, k), dtype=np.int8)
    assert (raw_dev(rk, wid, aq) == orc.matmul_i8_raw(aq, w1)).all()
    rk.rewrite_i8(wid, w2, s)
    assert (raw_dev(rk, wid, aq) == orc.matmul_i8_raw(aq, w2)).all()


def test_device_q8_0_packer_equals_gguf_blocks(rk, orc):
    # rk_pack_q8_0_f32 quantizes on the GPU with the llama.cpp rule; the
    # resident weight must equal the one packed from the oracle's blocks.
    note("pack_q8_0_f32 vs pack_q8_0")
    r = np.random.default_rng(21)
    m, k, n = 48, 384, 72
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[3, :32] = 0.0  # an all-zero block: scale 0, codes 0
    wq, wd = orc.q8_0_quantize(w)
    w1 = rk.pack_q8_0(orc.q8_0_blocks(wq, wd), n, k)
    w2 = rk.pack_q8_0_f32(w)
    eye = np.zeros((k, k), np.int8)
    np.fill_diagonal(eye, 1)
    # one-hot activations read the codes back exactly: c[i, j] = w_codes[j, i]
    assert (raw_dev(rk, w2, eye) == wq.T.astype(np.int32)).all()
    assert (raw_dev(rk, w1, eye) == raw_dev(rk, w2, eye)).all()
    # unit activation scales read the block scales back: c[i, j] = d[j, i/32]·code
    dq, ds = dev(rk, eye), dev(rk, np.ones((k, 1), np.float32))
    s1 = w8a8_dev(rk, w1, dq, ds, k, k, k)
    s2 = w8a8_dev(rk, w2, dq, ds, k, k, k)
    assert (s1 == s2).all()
    d32 = wd.view(np.float16).astype(np.float32)
    assert (s2 == (wq.astype(np.float32) * np.repeat(d32, 32, axis=1)).T).all()


def test_q8_0_blocks_split_on_the_device_keep_every_scale_exactly(rk, orc):
    # rk_pack_q8_0 uploads the 34-byte GGUF blocks once and splits them into
    # codes and f32 scales on the GPU (src/util/gguf.rs:125-200). Block scales
    # cover f16 subnormals, ±0, the largest finite value and negative values;
    # codes are random int8. One-hot activations with unit scale return
    # d·code exactly (an f16 times an int8 is exact in f32).
    note("device Q8_0 unpack: special scales")
    r = np.random.default_rng(31)
    n, k = 40, 256
    q = r.integers(-127, 128, (n, k), dtype=np.int8)
    d16 = (r.uniform(1e-4, 2.0, (n, k // 32))).astype(np.float16).view(np.uint16)
    special = np.array([0x0000, 0x8000, 0x0001, 0x03ff, 0x0200, 0x7bff, 0xbc00, 0x8001, 0x3c00], np.uint16)
    d16.reshape(-1)[:special.size] = special
    blocks = orc.q8_0_blocks(q, d16)
    wid = rk.pack_q8_0(blocks, n, k)
    eye = np.zeros((k, k), np.int8)
    np.fill_diagonal(eye, 1)
    assert (raw_dev(rk, wid, eye) == q.T.astype(np.int32)).all()
    dq, ds = dev(rk, eye), dev(rk, np.ones((k, 1), np.float32))
    got = w8a8_dev(rk, wid, dq, ds, k, k, k)
    want = (q.astype(np.float32) * np.repeat(orc.f16_to_f32(d16), 32, axis=1)).T
    assert (got == want).all()  # ±0 compare equal: the fold starts from +0
    # and through the real W8A8 path against the oracle's decode of the same blocks
    x = r.standard_normal((64, k)).astype(np.float32)
    aq, a_s = orc.quantize_rows(x, k)
    dqx, dsx = quantize_dev(rk, x, k)
    ref = orc.emu_matmul_gw(aq, a_s, k, q, orc.f16_to_f32(d16), 32)
    assert np.abs(w8a8_dev(rk, wid, dqx, dsx, k, 64, k) - ref).max() <= 1e-5 * np.abs(ref).max()


# Fused gate|up GEMM with the MLP glue in the epilogue: glue(gate·x, up·x)
# against the oracle's two W8A8 products and its glue (host.rs:12-39).
# Shapes select each tile configuration of the fused launch on a 256-CU
# MI355X: 2 / 224 / 256 tiles of 128x128 over the interleaved rows (n = 100
# also leaves padding rows in the last 16-row group).
@pytest.mark.parametrize("glu", ["silu", "gelu"])
@pytest.mark.parametrize("m,k,n", [(70, 512, 100), (1700, 256, 1024), (2048, 256, 1024)])
def test_w8a8_glu_fused(rk, orc, glu, m, k, n):
    r = np.random.default_rng(m + k + n + len(glu))
    x = r.standard_normal((m, k)).astype(np.float32)
    gate = (r.standard_normal((n, k)) * 0.05).astype(np.float32)
    up = (r.standard_normal((n, k)) * 0.05).astype(np.float32)
    gq, gd = orc.q8_0_quantize(gate)
    uq, ud = orc.q8_0_quantize(up)
    aq, a_s = orc.quantize_rows(x, k)
    f = lambda d: d.view(np.float16).astype(np.float32)
    g_ref = orc.emu_matmul_gw(aq, a_s, k, gq, f(gd), 32)
    u_ref = orc.emu_matmul_gw(aq, a_s, k, uq, f(ud), 32)
    ref = (orc.silu_mul if glu == "silu" else orc.gelu_mul)(g_ref, u_ref)
    kind = rk.GLU_SILU if glu == "silu" else rk.GLU_GELU
    dq, ds = quantize_dev(rk, x, k)
    lib = _lib(rk)
    for packer in ("blocks", "f32"):
        if packer == "blocks":
            wid = rk.pack_q8_0_glu(orc.q8_0_blocks(gq, gd), orc.q8_0_blocks(uq, ud), n, k)
        else:
            wid = rk.pack_q8_0_glu_f32(gate, up)
        for f16out in (False, True):
            note(f"W8A8 fused {glu} m={m} k={k} n={n} packer={packer} f16out={f16out}")
            dc = rk.DeviceBuffer(m * n * (2 if f16out else 4))
            rc = lib.rk_matmul_w8a8_glu_dev(int(wid), dq.ptr, ds.ptr, m, k, kind, dc.ptr, int(f16out), None)
            assert rc == 0, lib.rk_last_error()
            rk.synchronize()
            if f16out:
                got = dc.download((m, n), np.uint16).view(np.float16).astype(np.float32)
            else:
                got = dc.download((m, n), np.float32)
                assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()
            check(orc, got, ref)
            dc.free()
        # a fused weight is only accepted by the fused entry point, and vice versa
        dc = rk.DeviceBuffer(m * 2 * n * 4)
        assert lib.rk_matmul_w8a8_dev(int(wid), dq.ptr, ds.ptr, k, m, k, dc.ptr, None) == rk.RK_E_UNSUPPORTED
        dc.free()
    plain = rk.pack_q8_0(orc.q8_0_blocks(gq, gd), n, k)
    assert lib.rk_matmul_w8a8_glu_dev(int(plain), dq.ptr, ds.ptr, m, k, kind, None, 0, None) == rk.RK_E_UNSUPPORTED
