"""GPU parity of the host-buffer entry points and the driver-type mirrors
(`I8Context`, `RocketCtx`, `RocketFaCtx`), through the C ABI.

These are the paths an unchanged caller that keeps its tensors in host memory
takes: Clef's expert workers (I8Context::matmul_gw with codes, activation
scales and per-call weight scales, src/clef/engine_npu.rs:75-110), Clef's
vision tower (RocketCtx::matmul_prepacked and RocketFaCtx::flash_attn,
src/clef/vision/npu.rs:150-233) and every Flex `matmul` / `attention*`. Their
buffers move through page-locked staging in row chunks; at the config-2 size
(3633 rows) the product runs in several chunks, so these tests also cover the
chunk boundaries. Integer results are bit-exact; scaled f32 results are held
to 1e-5 of the largest value against `orc_emu_matmul_gw`."""
import sys

import numpy as np
import pytest

from burn_rocket import synth

pytestmark = pytest.mark.gpu
COS_MIN, REL_MAX = 0.9999, 1e-2


def note(msg):
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def check(orc, got, ref):
    assert orc.cosine(got, ref) >= COS_MIN
    assert orc.max_rel(got, ref) <= REL_MAX


@pytest.mark.parametrize("group", [32, 64, 128])
def test_i8context_matmul_gw_full_config2(rk, orc, group):
    # Clef's gw_matmul at the config-2 up-projection shape: codes and scales
    # quantized per row per group on the host side, the weight's codes packed
    # alone (pack_weight_gw) and its scales passed with each call.
    m, k, n = synth.W8A8["m"], synth.W8A8["hidden"], synth.W8A8["inter"]
    note(f"I8Context.matmul_gw m={m} k={k} n={n} group={group}")
    r = np.random.default_rng(group)
    x = r.standard_normal((m, k)).astype(np.float32)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    aq, a_s = orc.quantize_rows(x, group)
    wq, w_s = orc.quantize_rows(w, group)
    ctx = rk.I8Context.new_at(1, 0)
    wt = ctx.pack_weight_gw(128, k, n, np.zeros(n * k, np.int8), group)
    ctx.rewrite_weight_gw(wt, wq)
    cf = np.empty(m * n, np.float32)
    ctx.matmul_gw(m, k, n, aq, a_s, w_s, cf, wt)
    ref = orc.emu_matmul_gw(aq, a_s, group, wq, w_s, group)
    got = cf.reshape(m, n)
    check(orc, got, ref)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    # new codes in the same slot (the streamed-expert refill), other scales
    note(f"I8Context.rewrite_weight_gw + matmul_gw group={group}")
    wq2 = wq[::-1].copy()
    w_s2 = (w_s[::-1] * 1.5).astype(np.float32)
    ctx.rewrite_weight_gw(wt, wq2)
    ctx.matmul_gw(m, k, n, aq, a_s, w_s2, cf, wt)
    ref2 = orc.emu_matmul_gw(aq, a_s, group, wq2, w_s2, group)
    assert np.abs(cf.reshape(m, n) - ref2).max() <= 1e-5 * np.abs(ref2).max()


def test_i8context_raw_matmul_is_bit_exact_full_config2(rk, orc):
    # I8Context::matmul (int8.rs:606-640): per-channel weight, exact int32.
    m, k, n = synth.W8A8["m"], synth.W8A8["inter"], synth.W8A8["hidden"]
    note(f"I8Context.matmul raw m={m} k={k} n={n}")
    r = np.random.default_rng(7)
    a = r.integers(-127, 128, (m, k), dtype=np.int8)
    b = r.integers(-127, 128, (n, k), dtype=np.int8)
    ctx = rk.I8Context(1)
    wt = ctx.pack_weight(128, k, n, b)
    c = np.empty(m * n, np.int32)
    ctx.matmul(m, k, n, a, c, wt)
    assert (c.reshape(m, n) == orc.matmul_i8_raw(a, b)).all()


def test_matmul_i8_gw_resident_scales_equal_passed_scales(rk, orc):
    # b_scale NULL uses the scales packed with the weight: the same result as
    # passing those scales.
    note("rk_matmul_i8_gw resident vs passed scales")
    m, k, n, g = 100, 256, 96, 64
    r = np.random.default_rng(3)
    aq, a_s = orc.quantize_rows(r.standard_normal((m, k)).astype(np.float32), g)
    wq, w_s = orc.quantize_rows((r.standard_normal((n, k)) * 0.02).astype(np.float32), g)
    wid = rk.pack_i8_codes(wq, w_s, g)
    lib = rk.lib()
    outs = []
    for bs in (None, w_s):
        out = np.empty((m, n), np.float32)
        rc = lib.rk_matmul_i8_gw(int(wid), aq.ctypes.data, a_s.ctypes.data, None if bs is None else bs.ctypes.data,
                                 m, k, out.ctypes.data)
        assert rc == 0, lib.rk_last_error()
        outs.append(out)
    assert (outs[0] == outs[1]).all()
    ref = orc.emu_matmul_gw(aq, a_s, g, wq, w_s, g)
    assert np.abs(outs[0] - ref).max() <= 1e-5 * np.abs(ref).max()


def test_i8context_errors_follow_the_reference(rk):
    ctx = rk.I8Context(1)
    with pytest.raises(rk.RocketError) as e:
        ctx.pack_weight_gw(128, 64, 32, np.zeros(64 * 32, np.int8), 0)
    assert e.value.rc == rk.RK_E_SHAPE
    wt = ctx.pack_weight(128, 64, 32, np.zeros(64 * 32, np.int8))
    with pytest.raises(rk.RocketError) as e:
        ctx.matmul_gw(4, 64, 32, np.zeros(256, np.int8), np.ones(4, np.float32), np.ones(32, np.float32),
                      np.empty(128, np.float32), wt)
    assert e.value.rc == rk.RK_E_SHAPE
    with pytest.raises(rk.RocketError) as e:
        ctx.rewrite_weight_gw(wt, np.zeros(64 * 32, np.int8))
    assert e.value.rc == rk.RK_E_SHAPE


@pytest.mark.parametrize("kind", ["f16", "q8_0", "i8g64", "qat"])
def test_host_matmul_over_row_chunks_equals_the_device_path(rk, orc, kind):
    # rk_matmul at M=3633 runs in several staged row chunks; the rows of every
    # chunk equal the oracle (exact integer parts, fp16 / f32 gates).
    m = synth.W8A8["m"]
    k, n = (1024, 3072) if kind != "qat" else (3072, 1024)
    note(f"rk_matmul staged kind={kind} m={m} k={k} n={n}")
    r = np.random.default_rng(11)
    x = r.standard_normal((m, k)).astype(np.float32)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    if kind == "f16":
        wid = rk.pack(w)
        got = rk.matmul(x, wid)
        ref = orc.gemm_f16(x.astype(np.float16), w.astype(np.float16))
        ref = ref.astype(np.float16).astype(np.float32)
        check(orc, got, ref)
    elif kind == "q8_0":
        wq, wd = orc.q8_0_quantize(w)
        wid = rk.pack_q8_0(orc.q8_0_blocks(wq, wd), n, k)
        got = rk.matmul(x, wid)
        aq, a_s = orc.quantize_rows(x, 32)
        ref = orc.emu_matmul_gw(aq, a_s, 32, wq, wd.view(np.float16).astype(np.float32), 32)
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    elif kind == "i8g64":
        wid = rk.pack_i8(w, 64)
        got = rk.matmul(x, wid)
        aq, a_s = orc.quantize_rows(x, 64)
        wq, w_s = orc.quantize_rows(w, 64)
        ref = orc.emu_matmul_gw(aq, a_s, 64, wq, w_s, 64)
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    else:
        codes = r.integers(-127, 128, (n, k), dtype=np.int8)
        w_scale = (r.random(n) * 0.01 + 0.001).astype(np.float32)
        wid = rk.pack_qat(codes, w_scale, n, k, 0.05, 0.0)
        got = rk.matmul(x, wid)
        aq, rs = orc.quantize_static(x, 0.05)
        ref = orc.qat_epilogue(orc.matmul_i8_raw(aq, codes), rs, w_scale, 0.0)
        assert (got == ref).all()


def test_rocketctx_matmul_prepacked(rk, orc):
    # Clef's vision linears: fp16 host A, resident fp16 weight, fp16 host C.
    m, k, n = 2394, 1152, 4304
    note(f"RocketCtx.matmul_prepacked m={m} k={k} n={n}")
    r = np.random.default_rng(5)
    a = r.standard_normal((m, k)).astype(np.float16)
    b = (r.standard_normal((n, k)) * 0.02).astype(np.float16)
    ctx = rk.RocketCtx(4)
    wt = ctx.pack_weight(128, k, n, b)
    c = np.empty(m * n, np.float16)
    ctx.matmul_prepacked(m, k, n, a, c, wt)
    check(orc, c.reshape(m, n).astype(np.float32), orc.gemm_f16(a, b))
    seg = ctx.pack_weight_seg(128, k, [b[:1000], b[1000:]])
    c2 = np.empty(m * n, np.float16)
    ctx.matmul_prepacked(m, k, n, a, c2, seg)
    assert (c2 == c).all()


# Additive masks as the reference's builders make them (masks.rs:11-114),
# restated: 0 where the predicate keeps a key, -inf elsewhere.
def _mask(n_q, n_kv, keep):
    i = np.arange(n_q)[:, None]
    j = np.arange(n_kv)[None, :]
    return np.where(np.broadcast_to(keep(i, j), (n_q, n_kv)), np.float16(0), np.float16(-np.inf)).astype(np.float16)


MASK_CASES = [
    # name, n_q, n_kv, keep(i, j), (mode, window, q0, k0)
    ("causal", 96, 96, lambda i, j: j <= i, (1, -1, 0, 0)),
    ("window 5", 96, 96, lambda i, j: np.abs(i - j) <= 5, (2, 5, 0, 0)),
    ("causal window 7", 96, 96, lambda i, j: (j <= i) & (j > i - 7), (3, 7, 0, 0)),
    ("causal block q0=40", 48, 88, lambda i, j: j <= i + 40, (1, -1, 40, 0)),
    ("causal window block q0=64 k0=32 w=20", 40, 72,
     lambda i, j: (32 + j <= 64 + i) & (32 + j > 64 + i - 20), (3, 20, 64, 32)),
    ("window block q0=30 k0=10 w=12", 50, 70, lambda i, j: np.abs((30 + i) - (10 + j)) <= 12, (2, 12, 30, 10)),
    ("keys above the queries", 32, 64, lambda i, j: j <= i - 40, (1, -1, 0, 40)),
]


@pytest.mark.parametrize("case", MASK_CASES, ids=[c[0] for c in MASK_CASES])
def test_rocketfactx_additive_masks_equal_the_predicates(rk, case):
    name, n_q, n_kv, keep, (mode, window, q0, k0) = case
    note(f"RocketFaCtx.flash_attn mask {name}")
    h, kv, hd, dv = 4, 2, 72, 72
    r = np.random.default_rng(n_q + n_kv)
    q = r.standard_normal((h, n_q, hd)).astype(np.float16)
    k = r.standard_normal((kv, n_kv, hd)).astype(np.float16)
    v = r.standard_normal((kv, dv, n_kv)).astype(np.float16)
    fa = rk.RocketFaCtx(4)
    out = np.empty(h * n_q * dv, np.float16)
    fa.flash_attn(n_q, n_kv, hd, dv, h, kv, hd ** -0.5, 0.0, q, k, v, _mask(n_q, n_kv, keep), out)
    want = rk.flash_attn_f16(q, k, v, n_q, n_kv, hd, h, kv, hd ** -0.5, 0.0, mode, window, q0, k0, dv=dv)
    # The same visible keys per row; a mask may fit another mode of the same
    # intervals (a band with both ends inside the keys is also a causal
    # window), whose launch may split keys differently: equal to fp16 rounding.
    got, want = out.reshape(h, n_q, dv).astype(np.float32), want.astype(np.float32)
    assert np.abs(got - want).max() <= 2e-3 * max(1.0, np.abs(want).max())


def test_rocketfactx_rejects_masks_that_are_not_predicates(rk):
    h, kv, hd, n = 2, 1, 64, 32
    fa = rk.RocketFaCtx(1)
    q = np.zeros(h * n * hd, np.float16)
    k = np.zeros(kv * n * hd, np.float16)
    v = np.zeros(kv * hd * n, np.float16)
    out = np.empty(h * n * hd, np.float16)
    for bad in (np.full((n, n), -1.0, np.float16),                      # a finite bias
                _mask(n, n, lambda i, j: (j % 2) == 0),                  # rows of several intervals
                _mask(n, n, lambda i, j: (i % 2 == 0) | (j < 0)),        # full and empty rows alternate
                _mask(n, n, lambda i, j: j <= i // 2)):                  # a band that widens
        with pytest.raises(rk.RocketError) as e:
            fa.flash_attn(n, n, hd, hd, h, kv, 0.125, 0.0, q, k, v, bad, out)
        assert e.value.rc == rk.RK_E_UNSUPPORTED


def test_host_attention_reports_fp16_range(rk):
    # A q value beyond fp16's range: the reference's score surface saturates
    # and it answers Status::Range (-6); so does rk_attention.
    n, h, d = 16, 2, 64
    q = np.zeros((1, n, h * d), np.float32)
    q[0, 3, 5] = 1e6
    k = np.ones((1, n, h * d), np.float32)
    with pytest.raises(rk.RocketError) as e:
        rk.attention(q, k, k, h, h, d, d ** -0.5)
    assert e.value.rc == rk.RK_E_RANGE
    rk.attention(np.ones_like(q), k, k, h, h, d, d ** -0.5)  # in range: no error


def test_trim_scratch_keeps_the_just_used_set(rk):
    note("trim_scratch / mem_stats host_bytes")
    x = np.ones((64, 128), np.float32)
    wid = rk.pack(np.ones((32, 128), np.float32))
    rk.matmul(x, wid)
    ms = rk.mem_stats()
    assert ms.host_bytes > 0 and ms.n_scratch > 0
    rk.trim_scratch()            # marks the set in use until now
    a = np.ones(1000, np.float32)
    o = np.empty_like(a)
    assert rk.lib().rk_silu_mul(a.ctypes.data, a.ctypes.data, o.ctypes.data, a.size) == 0  # host entry: scratch "glue"
    rk.trim_scratch()            # frees what only the matmul used
    left = rk.mem_stats().n_scratch
    assert 0 < left < ms.n_scratch
    rk.clear_scratch()
    ms = rk.mem_stats()
    assert ms.scratch_bytes == 0 and ms.host_bytes == 0
    assert (rk.matmul(x, wid) == 128.0).all()  # allocated again on demand
