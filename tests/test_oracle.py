"""CPU tests that pin the oracle before it is trusted as the parity reference.

Every check here is independent of the oracle's own formula: the reference's
known-answer tests (cited), closed forms, exact integer arithmetic in numpy,
and brute force on tiny inputs.
"""
import numpy as np
import pytest


def _rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------ fp16 ----
def test_f16_round_trip_is_exact_for_every_f16(orc):
    h = np.arange(1 << 16, dtype=np.uint16)
    f = orc.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    same = (f.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(f) & np.isnan(ref))
    assert same.all()
    finite = ~np.isnan(ref)
    back = orc.f32_to_f16(f[finite])
    assert (back == h[finite]).all()


def test_f32_to_f16_is_round_to_nearest_even(orc):
    # numpy's float32 → float16 cast is IEEE RNE; compare on random values,
    # exact ties, subnormals, overflow and the largest finite boundaries.
    r = _rng(1)
    x = np.concatenate([
        r.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** r.integers(-9, 6, 200000),
        np.array([65504.0, 65519.0, 65520.0, 1e6, -1e6, 5.96e-8, 2.98e-8, 2.99e-8, 1e-10, 0.0, -0.0],
                 dtype=np.float32),
    ]).astype(np.float32)
    # exact halfway points between consecutive f16 values
    h = np.arange(0x0001, 0x7bff, 7, dtype=np.uint16).view(np.float16).astype(np.float32)
    h2 = (np.arange(0x0002, 0x7c00, 7, dtype=np.uint16)).view(np.float16).astype(np.float32)
    mid = ((h.astype(np.float64) + h2.astype(np.float64)) / 2).astype(np.float32)
    x = np.concatenate([x, mid, -mid])
    got = orc.f32_to_f16(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert (got == ref).all()


# ------------------------------------------------------------ quantizers ----
def test_quantizer_roundtrip_bound_group_max_and_zero_group(orc):
    # crates/burn-rocket/src/host.rs:189-222
    k, group = 128, 32
    r = _rng(2)
    x = r.uniform(-1, 1, k).astype(np.float32)
    x[70] = 9.5  # outlier in group 2
    q, s = orc.quantize_rows(x[None, :], group)
    q, s = q[0], s[0]
    for g in range(k // group):
        seg = x[g * group:(g + 1) * group]
        amax = np.abs(seg).max()
        assert abs(s[g] - amax / 127) <= 1e-9 * max(amax, 1)
        deq = q[g * group:(g + 1) * group].astype(np.float32) * s[g]
        assert (np.abs(seg - deq) <= s[g] * 0.5 + 1e-6).all()
    assert q[70] == 127
    assert s[2] > s[1]
    zq, zs = orc.quantize_rows(np.zeros((1, 32), np.float32), 32)
    assert zs[0, 0] > 0 and np.isfinite(zs[0, 0]) and (zq == 0).all()


def test_quantizer_is_round_half_away_of_x_times_inverse(orc):
    # src/clef/int8.rs:190-210: x·(1/s) and x/s differ only at exact .5 boundaries.
    r = _rng(3)
    x = (r.uniform(-1, 1, (4, 256)) * 5).astype(np.float32)
    q, s = orc.quantize_rows(x, 128)
    for row in range(4):
        for g in range(2):
            seg = x[row, g * 128:(g + 1) * 128]
            want = np.clip(np.round(seg.astype(np.float64) / s[row, g]), -127, 127)
            assert np.abs(q[row, g * 128:(g + 1) * 128] - want).max() <= 1
            assert (np.abs(q[row, g * 128:(g + 1) * 128]) == 127).any()
    # Half-away-from-zero, not ties-to-even: 2.5 → 3 and -2.5 → -3 at scale 1.
    x = np.zeros((1, 32), np.float32)
    x[0, :4] = [127.0, 2.5, -2.5, 0.5]
    q, s = orc.quantize_rows(x, 32)
    assert s[0, 0] == np.float32(1.0)
    assert list(q[0, :4]) == [127, 3, -3, 1]


def test_q8_0_block_dequant_kat(orc):
    # src/util/gguf.rs:250-262: scale 0.5, codes ff/00/01 → -0.5/0/0.5.
    raw = np.zeros(34, np.uint8)
    raw[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    raw[2], raw[3], raw[4] = 0xFF, 0x00, 0x01
    v = orc.q8_0_dequant(raw, 32)
    assert v[0] == -0.5 and v[1] == 0.0 and v[2] == 0.5


def test_q8_0_quantizes_against_the_stored_f16_scale(orc):
    # crates/rocket-npu/src/bin/q8_bench.rs:200-220
    r = _rng(4)
    w = (r.standard_normal((8, 96)) * 0.02).astype(np.float32)
    q, d = orc.q8_0_quantize(w)
    dval = d.view(np.float16).astype(np.float32)
    for row in range(8):
        for b in range(3):
            seg = w[row, b * 32:(b + 1) * 32]
            assert d[row, b] == np.float16(np.abs(seg).max() / np.float32(127)).view(np.uint16)
            inv = np.float32(1) / dval[row, b]
            want = np.clip(np.trunc(seg * inv + np.copysign(0.5, seg * inv)), -127, 127)
            assert (q[row, b * 32:(b + 1) * 32] == want).all()
    blocks = orc.q8_0_blocks(q, d)
    deq = orc.q8_0_dequant(blocks, w.size).reshape(w.shape)
    assert np.allclose(deq, q.astype(np.float32) * np.repeat(dval, 32, axis=1), rtol=0, atol=0)
    assert (np.abs(deq - w) <= np.repeat(dval, 32, axis=1) * 0.5 + 1e-7).all()


def test_static_code_rounds_ties_to_even_and_saturates(orc):
    # crates/burn-rocket/src/ext.rs:2257-2272
    x = np.array([[0.5, 1.5, 2.5, -0.5, -1.5, 1000.0, -1000.0]], np.float32)
    q, rs = orc.quantize_static(x, 1.0)
    assert list(q[0]) == [0, 2, 2, 0, -2, 127, -128] and rs[0] == 1.0
    scale = np.float32(0.0173)
    codes = np.array([-128, -77, -1, 0, 3, 64, 127], np.float32)
    q, _ = orc.quantize_static((codes * scale)[None, :], float(scale))
    assert list(q[0]) == list(codes.astype(int))
    # in_scale == 0 → per-row dynamic max(amax/127, 1e-12)
    x = np.array([[1.0, -2.54, 0.0]], np.float32)
    q, rs = orc.quantize_static(x, 0.0)
    assert rs[0] == np.float32(np.float32(2.54) / np.float32(127))


# ------------------------------------------------------- int8 products ----
def test_raw_int8_product_is_exact(orc):
    r = _rng(5)
    a = r.integers(-127, 128, (37, 160), dtype=np.int8)
    w = r.integers(-127, 128, (23, 160), dtype=np.int8)
    got = orc.matmul_i8_raw(a, w)
    assert (got == a.astype(np.int64) @ w.astype(np.int64).T).all()
    p = orc.i8_block_partials(a, w)
    ref = np.einsum("mbk,nbk->mnb", a.reshape(37, 5, 32).astype(np.int64), w.reshape(23, 5, 32).astype(np.int64))
    assert (p == ref).all()
    assert (p.sum(axis=2) == got).all()


def test_emulated_gw_matmul_has_an_exact_integer_part(orc):
    # src/clef/int8.rs:212-240: unit scales give the exact int64 dot.
    r = _rng(6)
    m, k, n, g = 7, 256, 5, 128
    aq = r.integers(-127, 128, (m, k), dtype=np.int8)
    wq = r.integers(-127, 128, (n, k), dtype=np.int8)
    got = orc.emu_matmul_gw(aq, np.ones((m, k // g), np.float32), g, wq, np.ones((n, k // g), np.float32), g)
    assert (got.astype(np.int64) == aq.astype(np.int64) @ wq.astype(np.int64).T).all()
    assert (orc.emu_matmul_gw(aq, np.ones((m, k // g), np.float32), g, wq, np.ones((n, k // g), np.float32), g,
                              threads=1) == got).all()


def test_emulated_gw_matmul_applies_scales_per_group(orc):
    # host.rs:225-276: int8 codes + per-row/per-group scales ≈ the f32 product.
    r = _rng(7)
    m, k, n, g = 8, 64, 8, 32
    a = (r.uniform(-1, 1, (m, k)) * 2).astype(np.float32)
    b = r.uniform(-1, 1, (n, k)).astype(np.float32)
    aq, a_s = orc.quantize_rows(a, g)
    bq, b_s = orc.quantize_rows(b, g)
    got = orc.emu_matmul_gw(aq, a_s, g, bq, b_s, g)
    want = a @ b.T
    assert (np.abs(got - want) <= 0.1 * np.maximum(np.abs(want), 1)).all()
    # Exact formula in f64 from the integer partials: a transposed or shifted
    # scale layout would be off by far more than f32 rounding.
    p = orc.i8_block_partials(aq, bq).astype(np.float64)
    exact = (p * (a_s[:, None, :].astype(np.float64) * b_s[None, :, :])).sum(axis=2)
    assert np.abs(got - exact).max() <= 1e-5 * np.abs(exact).max()


def test_per_token_activation_scale(orc):
    r = _rng(8)
    m, k, n = 16, 256, 24
    x = r.standard_normal((m, k)).astype(np.float32)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    xq, xs = orc.quantize_rows(x, k)
    wq, wd = orc.q8_0_quantize(w)
    ws = wd.view(np.float16).astype(np.float32)
    got = orc.emu_matmul_gw(xq, xs, k, wq, ws, 32)
    p = orc.i8_block_partials(xq, wq).astype(np.float64)
    exact = xs.astype(np.float64)[:, :, None][:, 0, :] * (p * ws[None, :, :]).sum(axis=2)
    assert np.abs(got - exact).max() <= 1e-5 * np.abs(exact).max()
    assert orc.cosine(got, x @ w.T) > 0.999


def test_qat_epilogue(orc):
    acc = np.array([[100, -200], [0, 7]], np.int64)
    rs = np.array([0.5, 2.0], np.float32)
    ws = np.array([0.1, 0.01], np.float32)
    y = orc.qat_epilogue(acc, rs, ws, 0.0)
    assert np.allclose(y, [[5.0, -1.0], [0.0, 0.14]], rtol=1e-6)
    y = orc.qat_epilogue(acc, rs, ws, 0.5)  # rounded to the 0.5 grid
    assert np.allclose(y, [[5.0, -1.0], [0.0, 0.0]])


# ------------------------------------------------------------- fp16 GEMM ----
def test_gemm_f16_closed_forms(orc):
    r = _rng(9)
    # identity: C = A exactly
    a = r.standard_normal((16, 64)).astype(np.float16)
    eye = np.eye(64, dtype=np.float16)
    assert (orc.gemm_f16(a, eye) == a.astype(np.float32)).all()
    # small integers: every partial sum is exact in f32
    a = r.integers(-8, 9, (9, 48)).astype(np.float16)
    b = r.integers(-8, 9, (11, 48)).astype(np.float16)
    assert (orc.gemm_f16(a, b) == (a.astype(np.int64) @ b.astype(np.int64).T)).all()
    # random: f32 accumulation within a few ulp-multiples of the f64 product
    a = r.standard_normal((33, 1024)).astype(np.float16)
    b = (r.standard_normal((17, 1024)) * 0.02).astype(np.float16)
    ref = a.astype(np.float64) @ b.astype(np.float64).T
    got = orc.gemm_f16(a, b)
    assert np.abs(got - ref).max() < 1e-4 * np.abs(ref).max()
    assert np.allclose(orc.gemm_f16_f64(a, b), ref, rtol=1e-12, atol=1e-12)


# ----------------------------------------------------------------- masks ----
def _keep_grid(orc, mode, w, n_q, n_kv, q0, k0):
    return np.array([[orc.mask_keep(mode, w, q0 + i, k0 + j) for j in range(n_kv)] for i in range(n_q)])


def test_mask_predicates_match_the_reference_builders(orc):
    # crates/burn-rocket/src/masks.rs:124-301
    t, j = np.meshgrid(np.arange(8), np.arange(8), indexing="ij")
    assert (_keep_grid(orc, 1, -1, 8, 8, 0, 0) == (j <= t)).all()
    assert (_keep_grid(orc, 2, 3, 8, 8, 0, 0) == (np.abs(t - j) <= 3)).all()
    assert (_keep_grid(orc, 3, 3, 8, 8, 0, 0) == ((j <= t) & (t - j < 3))).all()
    # block forms with offsets
    i, jj = np.meshgrid(np.arange(5), np.arange(7), indexing="ij")
    assert (_keep_grid(orc, 2, 3, 5, 7, 10, 8) == (np.abs((10 + i) - (8 + jj)) <= 3)).all()
    i, jj = np.meshgrid(np.arange(4), np.arange(10), indexing="ij")
    assert (_keep_grid(orc, 1, -1, 4, 10, 8, 4) == (4 + jj <= 8 + i)).all()
    i, jj = np.meshgrid(np.arange(5), np.arange(12), indexing="ij")
    k_ = _keep_grid(orc, 3, 4, 5, 12, 16, 8)
    assert (k_ == ((8 + jj <= 16 + i) & ((16 + i) - (8 + jj) < 4))).all()
    # keys above the chunk: fully masked; one-row overlap
    assert not _keep_grid(orc, 1, -1, 4, 8, 20, 24).any()
    # ragged 30k tail: visible run of row i is exactly q0 + i + 1
    n_kv, q0 = 29960, 29952
    for i in range(8):
        vis = sum(orc.mask_keep(1, -1, q0 + i, jj) for jj in range(q0 - 2, n_kv))
        assert vis == min(q0 + i + 1, n_kv) - (q0 - 2)
    # window 1 causal: only the diagonal
    assert (_keep_grid(orc, 3, 1, 6, 6, 0, 0) == np.eye(6, dtype=bool)).all()


# ------------------------------------------------------------- attention ----
def _qkv(r, n_q, n_kv, h, kv, d, sig=1.0):
    q = (r.standard_normal((n_q, h * d)) * sig).astype(np.float16)
    k = (r.standard_normal((n_kv, kv * d)) * sig).astype(np.float16)
    v = r.standard_normal((n_kv, kv * d)).astype(np.float16)
    return q, k, v


@pytest.mark.parametrize("fn", ["attention_ref", "attention_flex"])
def test_attention_single_visible_key_returns_that_value_row(orc, fn):
    # attn/oneshot.rs:763-805: a one-hot softmax returns the key's value exactly.
    r = _rng(10)
    n, h, kv, d = 6, 4, 2, 32
    q, k, v = _qkv(r, n, n, h, kv, d)
    out = getattr(orc, fn)(q, k, v, h, kv, d, 0.125, mode=3, window=1)  # t - 1 < j <= t
    for hh in range(h):
        g = hh // (h // kv)
        assert (out[:, hh * d:(hh + 1) * d] == v[:, g * d:(g + 1) * d].astype(np.float32)).all()


@pytest.mark.parametrize("fn", ["attention_ref", "attention_flex"])
def test_attention_closed_forms(orc, fn):
    r = _rng(11)
    n, h, kv, d = 9, 4, 2, 16
    q, k, v = _qkv(r, n, n, h, kv, d)
    f = getattr(orc, fn)
    # zero queries: uniform average of the visible prefix (causal) per kv head
    out = f(np.zeros_like(q), k, v, h, kv, d, 0.3, mode=1)
    vf = v.astype(np.float64)
    for hh in range(h):
        g = hh // 2
        cum = np.cumsum(vf[:, g * d:(g + 1) * d], axis=0) / np.arange(1, n + 1)[:, None]
        assert np.allclose(out[:, hh * d:(hh + 1) * d], cum, rtol=1e-5, atol=1e-5)
    # constant V: output is that constant whatever the scores
    vc = np.full_like(v, 0.75)
    out = f(q, k, vc, h, kv, d, 0.3, mode=0)
    assert np.allclose(out, 0.75, rtol=1e-6)
    # emptied rows (keys all above the chunk) average V over every key
    # (attn/oneshot.rs:909-944)
    out = f(q[:3], k, v, h, kv, d, 0.3, mode=1, q0=0, k0=5)
    for hh in range(h):
        g = hh // 2
        assert np.allclose(out[:, hh * d:(hh + 1) * d], vf[:, g * d:(g + 1) * d].mean(axis=0), rtol=1e-5,
                           atol=1e-5)


def test_attention_ref_matches_brute_force_softmax(orc):
    # Tiny brute force in numpy float64 (GQA head mapping, scale, softcap, mask).
    r = _rng(12)
    n_q, n_kv, h, kv, d = 5, 37, 8, 2, 64
    q, k, v = _qkv(r, n_q, n_kv, h, kv, d)
    for softcap in (0.0, 20.0):
        for mode, window in ((0, -1), (2, 2)):
            out = orc.attention_ref(q, k, v, h, kv, d, 0.125, softcap, mode, window, q0=30, k0=0)
            for hh in range(h):
                g = hh // (h // kv)
                qq = q[:, hh * d:(hh + 1) * d].astype(np.float64)
                kk = k[:, g * d:(g + 1) * d].astype(np.float64)
                vv = v[:, g * d:(g + 1) * d].astype(np.float64)
                s = (qq @ kk.T) * 0.125
                if softcap:
                    s = softcap * np.tanh(s / softcap)
                t = 30 + np.arange(n_q)[:, None]
                j = np.arange(n_kv)[None, :]
                if mode == 2:
                    s = np.where(np.abs(t - j) <= window, s, -np.inf)
                p = np.exp(s - s.max(axis=1, keepdims=True))
                want = (p / p.sum(axis=1, keepdims=True)) @ vv
                assert np.abs(out[:, hh * d:(hh + 1) * d] - want).max() < 2e-6


def test_attention_flex_online_fold_equals_one_pass(orc):
    # attn/mod.rs:1902-1990: the tiled online softmax equals one materialised pass.
    r = _rng(13)
    n, h, kv, d = 200, 4, 1, 72
    q, k, v = _qkv(r, n, n, h, kv, d)
    for mode, w in ((1, -1), (0, -1), (3, 50), (2, 17)):
        a = orc.attention_flex(q, k, v, h, kv, d, 72 ** -0.5, mode=mode, window=w)
        b = orc.attention_ref(q, k, v, h, kv, d, 72 ** -0.5, mode=mode, window=w)
        assert orc.cosine(a, b) > 0.999999
        assert np.abs(a - b).max() < 2e-5


# ------------------------------------------------------------------- MoE ----
def test_route_top_k_ties_and_renormalisation(orc):
    r = _rng(14)
    logits = r.standard_normal((64, 16)).astype(np.float32)
    logits[0, :] = 0.0  # all tied: ids 0..k-1
    logits[1, 5] = logits[1, 9] = 7.0  # tie between 5 and 9 at the top
    ids, wts = orc.route(logits, 4, True)
    assert list(ids[0]) == [0, 1, 2, 3]
    assert list(ids[1][:2]) == [5, 9]
    for t in range(64):
        p = np.exp(logits[t].astype(np.float64) - logits[t].max())
        p /= p.sum()
        order = sorted(range(16), key=lambda e: (-p[e], e))[:4]
        if t > 1:
            assert list(ids[t]) == order
        assert abs(wts[t].sum() - 1.0) < 1e-6
        assert np.allclose(wts[t], p[list(ids[t])] / p[list(ids[t])].sum(), rtol=1e-5)
    ids2, wts2 = orc.route(logits, 4, False)
    assert (ids2 == ids).all() and (wts2 <= wts + 1e-7).all()


def test_moe_emulation_against_a_naive_w8a8_reference(orc):
    # src/clef/engine/tests.rs:445-505: the emulated expert is within 2e-3 of
    # the peak of a naive f64 evaluation of the same W8A8 pipeline (x and act
    # quantized per row per 32-group, f64 dots of codes times scales, silu·up
    # formed in f32 from the f64 gate/up values), and within 5 % relative L2
    # of the unquantized expert.
    r = _rng(15)
    s, H, I, E, K = 12, 64, 32, 4, 2
    x = r.standard_normal((s, H)).astype(np.float32)
    ids, wts = orc.route(r.standard_normal((s, E)).astype(np.float32), K)
    gw = (r.standard_normal((E, I, H)) * 0.3).astype(np.float32)
    uw = (r.standard_normal((E, I, H)) * 0.3).astype(np.float32)
    dw = (r.standard_normal((E, H, I)) * 0.3).astype(np.float32)
    (gq, gs), (uq, us), (dq, ds) = (_moe_q8(orc, w) for w in (gw, uw, dw))
    y = orc.moe_experts(x, ids, wts, gq, gs, uq, us, dq, ds)

    def naive(aq, a_s, codes, sc):  # Σ_c aq·a_s·code·scale in f64
        a = aq.astype(np.float64) * np.repeat(a_s.astype(np.float64), 32, axis=1)
        w = codes.astype(np.float64) * np.repeat(sc.astype(np.float64), 32, axis=1)
        return a @ w.T

    silu32 = lambda z: z / (np.float32(1) + np.exp(-z))
    want = np.zeros((s, H))
    f64 = np.zeros((s, H))
    xq, xs = orc.quantize_rows(x, 32)
    for t in range(s):
        for j in range(K):
            e = ids[t, j]
            g = naive(xq[t:t + 1], xs[t:t + 1], gq[e], gs[e]).astype(np.float32)
            u = naive(xq[t:t + 1], xs[t:t + 1], uq[e], us[e]).astype(np.float32)
            aq, a_s = orc.quantize_rows(silu32(g) * u, 32)
            want[t] += wts[t, j] * naive(aq, a_s, dq[e], ds[e])[0]
            xx = x[t].astype(np.float64)
            gf, uf = gw[e].astype(np.float64) @ xx, uw[e].astype(np.float64) @ xx
            f64[t] += wts[t, j] * (dw[e].astype(np.float64) @ (gf / (1 + np.exp(-gf)) * uf))
    peak = np.abs(want).max()
    assert np.abs(y - want).max() <= 2e-3 * peak
    assert np.sqrt(((y - f64) ** 2).sum() / (f64 ** 2).sum()) < 0.05


def _moe_q8(orc, w):
    q, d = orc.q8_0_quantize(w.reshape(-1, w.shape[-1]))
    return q.reshape(w.shape), d.view(np.float16).astype(np.float32).reshape(*w.shape[:-1], -1)


def test_moe_quantizes_both_activations_per_32_group(orc):
    # The reference's expert workers quantize x and silu(g)·u per row per
    # 32-value group (src/clef/engine.rs:1005-1006, 1034-1035; engine_npu.rs:93).
    # A row whose first 32-group is ~1e4 times larger than the second keeps the
    # second group only under that scheme: one scale per row would round it to
    # zero codes. Expert 0's gate/up read only x's small group; its down
    # weights read only act's small group (act's first group is made large
    # through rows of gate/up that read x's large group). The f64 value of the
    # expert FFN is then matched within Q8_0 error, where a per-row scale would
    # give exactly 0.
    H, I, E, K = 64, 64, 2, 1
    r = _rng(21)
    x = np.zeros((3, H), np.float32)
    x[:, :32] = r.uniform(500, 1000, (3, 32)) * r.choice([-1, 1], (3, 32))
    x[:, 32:] = r.uniform(0.05, 0.1, (3, 32)) * r.choice([-1, 1], (3, 32))
    gate = np.zeros((E, I, H), np.float32)
    up = np.zeros((E, I, H), np.float32)
    down = np.zeros((E, H, I), np.float32)
    gate[0, :32, :32] = r.uniform(0.5, 1.0, (32, 32)) / 32   # act[:32] large, from x's large group
    up[0, :32, :32] = r.uniform(0.5, 1.0, (32, 32)) / 32
    gate[0, 32:, 32:] = r.uniform(0.5, 1.0, (32, 32))        # act[32:] small, from x's small group
    up[0, 32:, 32:] = r.uniform(0.5, 1.0, (32, 32))
    down[0, :, 32:] = r.uniform(-1, 1, (H, 32))               # y reads act's small group only
    gate[1], up[1], down[1] = 0.01, 0.01, 0.01
    ids = np.zeros((3, K), np.uint32)
    wts = np.ones((3, K), np.float32)
    (gq, gs), (uq, us), (dq, ds) = (_moe_q8(orc, w) for w in (gate, up, down))
    y = orc.moe_experts(x, ids, wts, gq, gs, uq, us, dq, ds)
    silu = lambda z: z / (1 + np.exp(-z))
    x64 = x.astype(np.float64)
    g = x64 @ gate[0].astype(np.float64).T
    u = x64 @ up[0].astype(np.float64).T
    want = (silu(g) * u) @ down[0].astype(np.float64).T
    assert np.abs(want).max() > 0.05  # the small groups carry the whole output
    assert np.abs(y - want).max() <= 3e-2 * np.abs(want).max()
    assert orc.cosine(y, want) > 0.999


def test_moe_experts_is_the_composition_of_the_pinned_primitives(orc):
    # orc_moe_experts = quantize_rows(group 32) → emu_matmul_gw (gate, up) →
    # silu·up → quantize_rows(group 32) → emu_matmul_gw (down) → ·router
    # weight → sum in ascending expert id; each primitive has its own KATs.
    r = _rng(22)
    s, H, I, E, K = 9, 96, 64, 5, 3
    x = r.standard_normal((s, H)).astype(np.float32)
    ids, wts = orc.route(r.standard_normal((s, E)).astype(np.float32), K)
    (gq, gs), (uq, us), (dq, ds) = (_moe_q8(orc, (r.standard_normal(shp) * 0.1).astype(np.float32))
                                    for shp in ((E, I, H), (E, I, H), (E, H, I)))
    y = orc.moe_experts(x, ids, wts, gq, gs, uq, us, dq, ds)
    xq, xs = orc.quantize_rows(x, 32)
    want = np.zeros((s, H), np.float32)
    for t in range(s):
        for j in np.argsort(ids[t], kind="stable"):
            e = ids[t, j]
            g = orc.emu_matmul_gw(xq[t:t + 1], xs[t:t + 1], 32, gq[e], gs[e], 32)
            u = orc.emu_matmul_gw(xq[t:t + 1], xs[t:t + 1], 32, uq[e], us[e], 32)
            act = orc.clef_silu_mul(g, u)
            aq, a_s = orc.quantize_rows(act, 32)
            want[t] += orc.emu_matmul_gw(aq, a_s, 32, dq[e], ds[e], 32)[0] * wts[t, j]
    assert (y == want).all()



def test_moe_experts_accumulates_onto_the_residual_in_expert_order(orc):
    # The reference's layer starts from the residual and adds each expert's
    # rows in ascending expert id (`let mut y = hid; … *a += b`,
    # src/clef/model.rs:606-614): y = ((hid + out_e0) + out_e1) + … . Each
    # slot's output alone comes from a top-1 call (0 + out = out exactly);
    # composing them onto hid in numpy in expert order must give the same
    # bits (a sum formed first and then added to hid rounds differently).
    r = _rng(24)
    s, H, I, E, K = 11, 64, 64, 6, 3
    x = r.standard_normal((s, H)).astype(np.float32)
    hid = (r.standard_normal((s, H)) * 3).astype(np.float32)
    ids, wts = orc.route(r.standard_normal((s, E)).astype(np.float32), K)
    (gq, gs), (uq, us), (dq, ds) = (_moe_q8(orc, (r.standard_normal(shp) * 0.1).astype(np.float32))
                                    for shp in ((E, I, H), (E, I, H), (E, H, I)))
    y = orc.moe_experts(x, ids, wts, gq, gs, uq, us, dq, ds, y0=hid)
    want = hid.copy()
    for j in np.argsort(ids, axis=1, kind="stable").T:
        sel = (np.arange(s), j)
        one = orc.moe_experts(x, ids[sel][:, None], wts[sel][:, None], gq, gs, uq, us, dq, ds)
        want = want + one
    assert (y == want).all()
    summed_first = hid + orc.moe_experts(x, ids, wts, gq, gs, uq, us, dq, ds)
    assert (y != summed_first).any()
    # onto zeros, the accumulating form is the overwriting one
    z = orc.moe_experts(x, ids, wts, gq, gs, uq, us, dq, ds, y0=np.zeros((s, H), np.float32))
    assert (z == orc.moe_experts(x, ids, wts, gq, gs, uq, us, dq, ds)).all()

def test_clef_silu_mul_formula(orc):
    # src/clef/model.rs:491-493: silu(v) = v / (1 + e^-v), then ·u, in f32;
    # against the same expression in f64 (within f32 rounding), its limits,
    # and silu(0)·u = 0.
    r = _rng(23)
    g = (r.standard_normal(4096) * 6).astype(np.float32)
    u = r.standard_normal(4096).astype(np.float32)
    got = orc.clef_silu_mul(g, u)
    g64 = g.astype(np.float64)
    want = g64 / (1 + np.exp(-g64)) * u
    assert np.abs(got - want).max() <= 4 * 2.0 ** -24 * np.abs(want).max()
    big = np.array([40.0, -40.0, 0.0], np.float32)
    out = orc.clef_silu_mul(big, np.ones(3, np.float32))
    assert out[0] == np.float32(40.0) and abs(out[1]) < 1e-15 and out[2] == 0.0


# ---- MLP glue (host.rs:12-39) ----------------------------------------------

def _gelu_composite(x):
    """Burn's gelu_approximate composite with powf, in f32 (host.rs:96-102)."""
    x = np.asarray(x, np.float32)
    inner = x + np.power(x, np.float32(3.0)) * np.float32(0.044715)
    inner = inner * np.float32(np.sqrt(2.0 / np.pi))
    return (x * (np.tanh(inner.astype(np.float64)).astype(np.float32) + np.float32(1.0))) * np.float32(0.5)


def test_gelu_tanh_matches_the_composite(orc):
    # host.rs:104-115: -30..30 in steps of 0.05, within 1e-6·max(|want|, 1)
    xs = (np.arange(-600, 601) * 0.05).astype(np.float32)
    got, want = orc.gelu_tanh(xs), _gelu_composite(xs)
    assert (np.abs(got - want) <= 1e-6 * np.maximum(np.abs(want), 1.0)).all()
    # gelu(x) - gelu(-x) = x (tanh is odd) and gelu(0) = 0
    assert np.abs((got - orc.gelu_tanh(-xs)) - xs).max() <= 4e-6 * np.abs(xs).max()
    assert orc.gelu_tanh(np.zeros(1, np.float32))[0] == 0.0


def test_gelu_mul_and_silu_mul_known_answers(orc):
    # host.rs:117-144 (same gate/up vectors)
    gate = np.array([0.0, 1.0, -1.0, 3.7, -12.5], np.float32)
    up = np.array([2.0, -1.0, 0.5, 0.25, 8.0], np.float32)
    assert (orc.gelu_mul(gate, up) == orc.gelu_tanh(gate) * up).all()
    want = gate.astype(np.float64) / (1.0 + np.exp(-gate.astype(np.float64))) * up
    got = orc.silu_mul(gate, up)
    assert (np.abs(got - want) <= 1e-6 * np.maximum(np.abs(want), 1.0)).all()
    # limits: silu(g)·u → g·u for large g, → 0 for very negative g; silu(0) = 0
    big = np.array([30.0, -30.0, 0.0], np.float32)
    assert np.allclose(orc.silu_mul(big, np.ones(3, np.float32)), [30.0, 0.0, 0.0], atol=1e-9)


def test_bf16_round_to_nearest_even(orc):
    import torch
    r = _rng(16)
    x = np.concatenate([r.standard_normal(4096).astype(np.float32) * 10,
                        # exact ties (low 16 bits 0x8000), both parities, and signed zero
                        (np.arange(64, dtype=np.uint32) * 0x10000 + 0x3F808000).view(np.float32),
                        np.array([0.0, -0.0, 65504.0, 1e-40, -3.0e38], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = orc.f32_to_bf16(x)
    assert (got == want).all()
    assert (orc.bf16_to_f32(got) == torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy()).all()


def test_rms_norm_known_answer_and_invariants(orc):
    # host.rs:146-162: x = [1, 2, 3, 4], w = [1, 0.5, 2, -1], eps = 1e-6
    x = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    w = np.array([1.0, 0.5, 2.0, -1.0], np.float32)
    inv = np.float32(1.0) / np.sqrt(np.float32(30.0 / 4.0) + np.float32(1e-6))
    assert (np.abs(orc.rms_norm(x, w, 1e-6) - x * inv * w) < 1e-6).all()
    assert (np.abs(orc.rms_norm(x, None, 1e-6) - x * inv) < 1e-6).all()
    # against an f64 evaluation over random rows (a dropped eps, a sum over the
    # wrong axis, or a weight applied per row instead of per column fail here)
    r = _rng(31)
    xs = r.standard_normal((37, 200)).astype(np.float32) * 3
    ws = r.standard_normal(200).astype(np.float32)
    x64 = xs.astype(np.float64)
    want = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-5) * ws
    assert np.abs(orc.rms_norm(xs, ws, 1e-5) - want).max() <= 1e-5 * np.abs(want).max()
    # eps = 0 and w = 1: each row then has mean square 1
    y = orc.rms_norm(xs, None, 0.0).astype(np.float64)
    assert np.abs((y * y).mean(axis=1) - 1.0).max() < 1e-5
    # eps dominates a tiny row: out ≈ x / sqrt(eps)
    tiny = np.full((1, 8), 1e-6, np.float32)
    assert np.allclose(orc.rms_norm(tiny, None, 1.0), tiny, rtol=1e-6)


def test_rope_known_answer_and_rotation(orc):
    # host.rs:164-177: half = 3 with these cos/sin, checked element by element
    x = np.array([1.0, 2.0, 3.0, -1.0, 0.5, 4.0], np.float32).reshape(1, 1, 1, 6)
    cos = np.array([[1.0, 0.5, -0.25]], np.float32)
    sin = np.array([[0.0, 0.5, 0.75]], np.float32)
    got = orc.rope(x, cos, sin).ravel()
    x1, x2 = x.ravel()[:3], x.ravel()[3:]
    assert (got[:3] == x1 * cos[0] - x2 * sin[0]).all()
    assert (got[3:] == x2 * cos[0] + x1 * sin[0]).all()
    # as a complex product (x1 + i·x2)·(cos + i·sin) per pair, the table row
    # picked by the position axis of [B, S, H, D]
    r = _rng(32)
    b, s, h, d = 2, 5, 3, 16
    xs = r.standard_normal((b, s, h, d)).astype(np.float32)
    ang = r.uniform(-4, 4, (s, d // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    z = (xs[..., :d // 2] + 1j * xs[..., d // 2:].astype(np.float64)) * \
        (cs[None, :, None, :] + 1j * sn[None, :, None, :].astype(np.float64))
    want = np.concatenate([z.real, z.imag], axis=-1)
    got = orc.rope(xs, cs, sn)
    assert np.abs(got - want).max() < 1e-5
    # a rotation keeps each pair's length; cos = 1, sin = 0 is the identity
    n_in = xs[..., :d // 2] ** 2 + xs[..., d // 2:] ** 2
    n_out = got[..., :d // 2] ** 2 + got[..., d // 2:] ** 2
    assert np.allclose(n_in, n_out, rtol=1e-5, atol=1e-6)
    ident = orc.rope(xs, np.ones((s, d // 2), np.float32), np.zeros((s, d // 2), np.float32))
    assert (ident == xs).all()
