"""GPU parity of the fused GQA flash attention (K3) against the oracle.

The oracle computes any subset of query rows exactly (rows are independent and
positions are absolute via q0), so full-size runs are checked on slices of
rows from the start, middle and end of the sequence. Gate: cosine >= 0.9999
and max relative error <= 1e-2 against the f32 tiled restatement of the Burn
CPU attention and the f64 flash_attn_ref restatement."""
import sys

import numpy as np
import pytest

from burn_rocket import synth

pytestmark = pytest.mark.gpu
COS_MIN, REL_MAX = 0.9999, 1e-2


def note(msg):
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def attn_dev(rk, q, k, v, h, kv, d, scale, softcap=0.0, mode=0, window=-1, q0=0, k0=0):
    n_q, n_kv = q.shape[0], k.shape[0]
    bufs = [rk.DeviceBuffer.from_array(np.ascontiguousarray(a).view(np.uint16)) for a in (q, k, v)]
    out = rk.DeviceBuffer(n_q * h * d * 2)
    rc = rk.lib().rk_attention_dev(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, n_q, n_kv, h, kv, d, scale, softcap, mode,
                                   window, q0, k0, out.ptr, None)
    assert rc == 0, rk.lib().rk_last_error()
    rk.synchronize()
    return out.download((n_q, h * d), np.uint16).view(np.float16).astype(np.float32)


def check(orc, got, ref):
    assert np.isfinite(got).all()
    cos, rel = orc.cosine(got, ref), orc.max_rel(got, ref)
    assert cos >= COS_MIN and rel <= REL_MAX, (cos, rel)


def check_rows(orc, got, q, k, v, h, kv, d, scale, rows, softcap=0.0, mode=0, window=-1, q0=0, k0=0,
               ref64=True):
    for a, b in rows:
        flex = orc.attention_flex(q[a:b], k, v, h, kv, d, scale, softcap, mode, window, q0 + a, k0)
        check(orc, got[a:b], flex)
        if ref64:
            ref = orc.attention_ref(q[a:b], k, v, h, kv, d, scale, softcap, mode, window, q0 + a, k0)
            check(orc, got[a:b], ref)


def _slices(n, w=48):
    return [(0, min(w, n)), (max(0, n // 2 - w // 2), min(n, n // 2 + w // 2)), (max(0, n - w), n)]


def test_config3_causal_gqa_full(rk, orc):
    c = synth.GQA_CAUSAL
    s, h, kv, d = c["s"], c["n_head"], c["n_kv"], c["d"]
    seeds = synth.SEEDS["gqa"]
    note(f"causal GQA S={s} H={h} KV={kv} D={d}")
    q = synth.normal_f16(seeds[0], (s, h * d))
    k = synth.normal_f16(seeds[1], (s, kv * d))
    v = synth.normal_f16(seeds[2], (s, kv * d))
    got = attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, mode=1)
    check_rows(orc, got, q, k, v, h, kv, d, d ** -0.5, _slices(s), mode=1)


def test_config4_bidirectional_mha_d72_full(rk, orc):
    c = synth.VISION
    s, h, d = c["s"], c["n_head"], c["d"]
    seeds = synth.SEEDS["vision"]
    note(f"bidirectional MHA S={s} H={h} D={d}")
    q = synth.normal_f16(seeds[6], (s, h * d))
    k = synth.normal_f16(seeds[7], (s, h * d))
    v = synth.normal_f16(seeds[8], (s, h * d))
    got = attn_dev(rk, q, k, v, h, h, d, d ** -0.5, mode=0)
    check_rows(orc, got, q, k, v, h, h, d, d ** -0.5, _slices(s, 32))


def test_config5_gqa_32_4_full(rk, orc):
    c = synth.MOE
    s, h, kv, d = c["s"], c["attn_heads"], c["attn_kv"], c["attn_d"]
    seeds = synth.SEEDS["moe"]
    note(f"causal GQA S={s} H={h} KV={kv} D={d}")
    q = synth.normal_f16(seeds[6], (s, h * d))
    k = synth.normal_f16(seeds[7], (s, kv * d))
    v = synth.normal_f16(seeds[8], (s, kv * d))
    got = attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, mode=1)
    check_rows(orc, got, q, k, v, h, kv, d, d ** -0.5, _slices(s, 64), mode=1)


@pytest.mark.parametrize("d", [32, 48, 64, 72, 80, 96, 112, 128, 256])
@pytest.mark.parametrize("h,kv", [(4, 4), (8, 2), (16, 2), (6, 3)])
def test_head_dims_and_groups(rk, orc, d, h, kv):
    note(f"attention d={d} h={h} kv={kv}")
    r = np.random.default_rng(d * 31 + h)
    n_q, n_kv = 150, 150
    q = r.standard_normal((n_q, h * d)).astype(np.float16)
    k = r.standard_normal((n_kv, kv * d)).astype(np.float16)
    v = r.standard_normal((n_kv, kv * d)).astype(np.float16)
    for mode in (0, 1):
        got = attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, mode=mode)
        check(orc, got, orc.attention_ref(q, k, v, h, kv, d, d ** -0.5, mode=mode))


@pytest.mark.parametrize("d", [32, 48, 64, 72, 80])
@pytest.mark.parametrize("h,kv", [(4, 4), (8, 2), (6, 3), (16, 16)])
def test_192_row_tiles(rk, orc, d, h, kv, monkeypatch):
    """Head dims up to 80 also run on 192-row query tiles (6 waves per key
    group), the default for unmasked calls whose 128-row grid needs an extra
    round on the CUs; forced here for every mask mode, ragged query and key
    counts and a softcap."""
    monkeypatch.setenv("RK_ATTN_ROWS", "192")
    r = np.random.default_rng(d * 17 + h + kv)
    n_q, n_kv = 407, 390
    q = r.standard_normal((n_q, h * d)).astype(np.float16)
    k = r.standard_normal((n_kv, kv * d)).astype(np.float16)
    v = r.standard_normal((n_kv, kv * d)).astype(np.float16)
    for mode, window, softcap in ((0, -1, 0.0), (1, -1, 0.0), (2, 25, 0.0), (3, 60, 0.0), (0, -1, 20.0)):
        note(f"192-row tiles d={d} h={h} kv={kv} mode={mode} window={window} softcap={softcap}")
        got = attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, softcap=softcap, mode=mode, window=window)
        check(orc, got, orc.attention_ref(q, k, v, h, kv, d, d ** -0.5, softcap, mode, window))


@pytest.mark.parametrize("d", [72, 80])
@pytest.mark.parametrize("rows,split", [("128", "1"), ("192", "1"), ("128", "2")])
def test_mixed_slot_equals_separate_slots(rk, orc, d, rows, split, monkeypatch):
    """Head dims 72 and 80 run the steady-state MFMA slots with the PV and
    Sᵀ products interleaved (RK_ATTN_MIX, default on); the sums are the same
    MFMAs in the same order per accumulator, so the output equals the separate
    slots bit for bit: 128- and 192-row tiles, the key split, every mask
    mode, key ranges of one to many tiles per group (the mixed loop runs only
    from the second tile of a group on)."""
    monkeypatch.setenv("RK_ATTN_ROWS", rows)
    monkeypatch.setenv("RK_ATTN_SPLIT", split)
    r = np.random.default_rng(d + int(rows) + int(split))
    h, kv = 8, 4
    for n_q, n_kv, mode, window in ((300, 450, 0, -1), (300, 300, 1, -1), (200, 200, 3, 70), (130, 60, 0, -1),
                                    (90, 130, 2, 40)):
        note(f"mixed slot d={d} rows={rows} split={split} n_q={n_q} n_kv={n_kv} mode={mode}")
        q = r.standard_normal((n_q, h * d)).astype(np.float16)
        k = r.standard_normal((n_kv, kv * d)).astype(np.float16)
        v = r.standard_normal((n_kv, kv * d)).astype(np.float16)
        outs = []
        for mix in ("1", "0"):
            monkeypatch.setenv("RK_ATTN_MIX", mix)
            outs.append(attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, mode=mode, window=window))
        assert (outs[0] == outs[1]).all()
        check(orc, outs[0], orc.attention_ref(q, k, v, h, kv, d, d ** -0.5, 0.0, mode, window))


@pytest.mark.parametrize("mode,window,n_q,n_kv,q0,k0", [
    (2, 17, 200, 200, 0, 0),      # band
    (3, 33, 200, 200, 0, 0),      # causal sliding window
    (1, -1, 64, 300, 236, 0),     # causal query chunk against its key prefix
    (3, 40, 64, 104, 400, 360),   # causal window chunk, keys start at q0 - window
    (2, 20, 50, 90, 300, 280),    # band chunk
    (1, -1, 40, 70, 10, 30),      # keys above the first rows: emptied rows average V
    (2, 5, 30, 40, 100, 0),       # band entirely outside the keys: every row emptied
    (0, -1, 1, 1, 0, 0),          # one query, one key
    (1, -1, 1, 129, 128, 0),      # one query, ragged key count
])
def test_mask_modes_and_block_offsets(rk, orc, mode, window, n_q, n_kv, q0, k0):
    note(f"mask mode={mode} w={window} n_q={n_q} n_kv={n_kv} q0={q0} k0={k0}")
    r = np.random.default_rng(n_q * 7 + n_kv)
    h, kv, d = 8, 2, 128
    q = r.standard_normal((n_q, h * d)).astype(np.float16)
    k = r.standard_normal((n_kv, kv * d)).astype(np.float16)
    v = r.standard_normal((n_kv, kv * d)).astype(np.float16)
    got = attn_dev(rk, q, k, v, h, kv, d, 0.0884, mode=mode, window=window, q0=q0, k0=k0)
    ref = orc.attention_ref(q, k, v, h, kv, d, 0.0884, 0.0, mode, window, q0, k0)
    check(orc, got, ref)


@pytest.mark.parametrize("split", ["1", "2"])
@pytest.mark.parametrize("d,h,kv,mode,window,softcap,n_q,n_kv,q0,k0", [
    (128, 8, 2, 1, -1, 0.0, 300, 300, 0, 0),     # causal: halves of unequal length per tile
    (64, 4, 4, 0, -1, 0.0, 200, 64, 0, 0),       # one key tile: the second half walks none
    (72, 16, 16, 0, -1, 0.0, 150, 150, 0, 0),    # padded head dim (row sums from the ones row of Vᵀ)
    (256, 3, 1, 2, 100, 0.0, 260, 260, 0, 0),    # two Oᵀ chunks per query tile, band
    (128, 8, 2, 1, -1, 0.0, 40, 70, 10, 30),     # emptied rows sweep every key in both halves
    (96, 6, 3, 3, 40, 15.0, 180, 180, 0, 0),     # causal window with a softcap
    (112, 8, 8, 2, 5, 0.0, 30, 40, 100, 0),      # every row emptied
])
def test_key_split(rk, orc, monkeypatch, split, d, h, kv, mode, window, softcap, n_q, n_kv, q0, k0):
    """RK_ATTN_SPLIT=2 splits every launch's key tiles between two workgroups
    (the second to finish merges the two partial softmax states, in split
    order); 1 never splits. Both against the oracle, and each bit-identical
    from one call to the next."""
    note(f"key split={split} d={d} h={h} kv={kv} mode={mode} w={window} cap={softcap} "
         f"n_q={n_q} n_kv={n_kv} q0={q0} k0={k0}")
    monkeypatch.setenv("RK_ATTN_SPLIT", split)
    r = np.random.default_rng(d + h * 3 + n_q + n_kv)
    q = r.standard_normal((n_q, h * d)).astype(np.float16)
    k = r.standard_normal((n_kv, kv * d)).astype(np.float16)
    v = r.standard_normal((n_kv, kv * d)).astype(np.float16)
    args = dict(softcap=softcap, mode=mode, window=window, q0=q0, k0=k0)
    got = attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, **args)
    again = attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, **args)
    assert (got == again).all()
    check(orc, got, orc.attention_ref(q, k, v, h, kv, d, d ** -0.5, softcap, mode, window, q0, k0))


@pytest.mark.parametrize("forced", ["", "7", "200"])
@pytest.mark.parametrize("mode,window", [(1, -1), (3, 300)])
def test_key_split_of_the_longest_causal_tiles(rk, orc, monkeypatch, forced, mode, window):
    """A causal grid of one round splits only its longest query tiles (the first
    n_split in dispatch order) and runs the rest whole in the same launch; the
    default count and forced ones (RK_ATTN_SPLIT_TILES), odd included."""
    note(f"partial key split mode={mode} window={window} forced={forced or 'default'}")
    monkeypatch.setenv("RK_ATTN_SPLIT_TILES", forced)
    r = np.random.default_rng(1000 + mode)
    n, h, kv, d = 1000, 32, 16, 64  # 16 query tiles of 64 × 16 kv heads = 256 tiles
    q = r.standard_normal((n, h * d)).astype(np.float16)
    k = r.standard_normal((n, kv * d)).astype(np.float16)
    v = r.standard_normal((n, kv * d)).astype(np.float16)
    got = attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, mode=mode, window=window)
    again = attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, mode=mode, window=window)
    assert (got == again).all()
    check_rows(orc, got, q, k, v, h, kv, d, d ** -0.5, _slices(n, 40) + [(600, 640), (960, 1000)], mode=mode,
               window=window, ref64=False)


@pytest.mark.parametrize("mode,window,softcap,q0,k0,n_q,n_kv", [
    (2, 512, 0.0, 0, 0, 1200, 1200),       # sliding layer, one chunk
    (0, -1, 0.0, 0, 0, 700, 700),          # full layer
    (2, 512, 0.0, 1024, 512, 176, 688),    # sliding layer, a later query chunk (keys from q0 - window)
    (3, 100, 30.0, 0, 0, 333, 333),        # causal window with a softcap
])
def test_head_dim_256_gemma_layers(rk, orc, mode, window, softcap, q0, k0, n_q, n_kv):
    """EmbeddingGemma's attention: 3 query heads on 1 kv head of 256 values
    (src/gemma/embeddinggemma/model.rs:165-230 calls attention_window and
    attention_window_block with its sliding window). Head dims above 128 run
    32-key tiles and two 128-row Oᵀ chunks per query tile."""
    note(f"d=256 gemma mode={mode} window={window} softcap={softcap} q0={q0} k0={k0} n_q={n_q} n_kv={n_kv}")
    r = np.random.default_rng(n_q + n_kv + mode)
    h, kv, d = 3, 1, 256
    q = r.standard_normal((n_q, h * d)).astype(np.float16)
    k = r.standard_normal((n_kv, kv * d)).astype(np.float16)
    v = r.standard_normal((n_kv, kv * d)).astype(np.float16)
    got = attn_dev(rk, q, k, v, h, kv, d, 1.0 / 16, softcap=softcap, mode=mode, window=window, q0=q0, k0=k0)
    rows = _slices(n_q, 48)
    check_rows(orc, got, q, k, v, h, kv, d, 1.0 / 16, rows, softcap=softcap, mode=mode, window=window,
               q0=q0, k0=k0)


@pytest.mark.parametrize("mode,window", [(0, -1), (2, 512)])
def test_gemma_attention_at_the_bench_size(rk, orc, mode, window):
    """EmbeddingGemma's attention at the measured size (2587 tokens, 3 query heads
    on 1 kv head of 256, full and 512-key sliding layers; key split on by
    default at this grid), on row slices from the start, middle and end, and
    bit-identical from one call to the next."""
    c = synth.GEMMA_TEXT
    s, h, kv, d = c["s"], c["n_head"], c["n_kv"], c["d"]
    note(f"gemma bench size S={s} mode={mode} window={window}")
    seeds = synth.SEEDS["gemma"]
    q = synth.normal_f16(seeds[0], (s, h * d))
    k = synth.normal_f16(seeds[1], (s, kv * d))
    v = synth.normal_f16(seeds[2], (s, kv * d))
    got = attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, mode=mode, window=window)
    assert (got == attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, mode=mode, window=window)).all()
    check_rows(orc, got, q, k, v, h, kv, d, d ** -0.5, _slices(s, 48), mode=mode, window=window)


def test_softcap(rk, orc):
    note("softcap 20")
    r = np.random.default_rng(99)
    h, kv, d, n = 8, 4, 64, 190
    q = (r.standard_normal((n, h * d)) * 3).astype(np.float16)
    k = (r.standard_normal((n, kv * d)) * 3).astype(np.float16)
    v = r.standard_normal((n, kv * d)).astype(np.float16)
    got = attn_dev(rk, q, k, v, h, kv, d, 0.125, softcap=20.0, mode=1)
    check(orc, got, orc.attention_ref(q, k, v, h, kv, d, 0.125, 20.0, 1))


def test_host_api_and_head_major_layout(rk, orc):
    note("rk_attention host f32 + rk_flash_attn_f16 head-major")
    r = np.random.default_rng(5)
    h, kv, d, n = 8, 2, 128, 97
    q = r.standard_normal((1, n, h * d)).astype(np.float32)
    k = r.standard_normal((1, n, kv * d)).astype(np.float32)
    v = r.standard_normal((1, n, kv * d)).astype(np.float32)
    out = rk.attention(q, k, v, h, kv, d, d ** -0.5, None, True)
    assert out.shape == (1, n, h * d)
    q16, k16, v16 = (orc.f32_to_f16(a[0]) for a in (q, k, v))
    ref = orc.attention_ref(q16, k16, v16, h, kv, d, d ** -0.5, 0.0, 1)
    check(orc, out[0], ref)
    # head-major: q [H][n][D], k [KV][n][D], v [KV][D][n]
    qh = q16.view(np.float16).reshape(n, h, d).transpose(1, 0, 2)
    kh = k16.view(np.float16).reshape(n, kv, d).transpose(1, 0, 2)
    vh = v16.view(np.float16).reshape(n, kv, d).transpose(1, 2, 0)
    oh = rk.flash_attn_f16(qh, kh, vh, n, n, d, h, kv, d ** -0.5, 0.0, 1)
    assert (oh.transpose(1, 0, 2).reshape(n, h * d).astype(np.float32) == out[0]).all()
    # window < 0 in the window modes means no window (ext.rs:99-126)
    a = rk.attention_window(q, k, v, h, kv, d, d ** -0.5, None, -1)
    b = rk.attention(q, k, v, h, kv, d, d ** -0.5, None, False)
    assert (a == b).all()
    a = rk.attention_causal_window(q, k, v, h, kv, d, d ** -0.5, None, -1)
    assert (a == out).all()


@pytest.mark.parametrize("mode", [0, 1])
def test_flash_attn_clef_padded_layout(rk, orc, mode):
    """The reference's padded head-major call (src/clef/vision/npu.rs:211-230):
    72-wide heads with q and k zero-padded to head_dim 96 and Vᵀ padded to dv 80
    rows, scale 72^-0.5. The first 72 output columns are the attention of the
    72-wide data (gates against both oracles), columns 72..79 are exactly zero."""
    s, h, d, dk, dvp = 301, 4, 72, 96, 80
    r = np.random.default_rng(96 + mode)
    q = r.standard_normal((s, h * d)).astype(np.float16)
    k = r.standard_normal((s, h * d)).astype(np.float16)
    v = r.standard_normal((s, h * d)).astype(np.float16)
    note(f"flash_attn head_dim {dk} dv {dvp} (72-wide data), mode {mode}")

    def pad_heads(x, w):  # [s, h·d] → [h][s][w], zero columns d..w
        out = np.zeros((h, s, w), np.float16)
        out[:, :, :d] = x.reshape(s, h, d).transpose(1, 0, 2)
        return out

    vt = np.zeros((h, dvp, s), np.float16)  # [h][dv][s], zero rows d..dv
    vt[:, :d, :] = v.reshape(s, h, d).transpose(1, 2, 0)
    o = rk.flash_attn_f16(pad_heads(q, dk), pad_heads(k, dk), vt, s, s, dk, h, h, d ** -0.5, 0.0, mode,
                          dv=dvp)
    assert o.shape == (h, s, dvp)
    assert (o[:, :, d:] == 0).all()
    got = o[:, :, :d].transpose(1, 0, 2).reshape(s, h * d).astype(np.float32)
    check(orc, got, orc.attention_ref(q, k, v, h, h, d, d ** -0.5, 0.0, mode))
    check(orc, got, orc.attention_flex(q, k, v, h, h, d, d ** -0.5, 0.0, mode))
    # dv above head_dim: q and k are padded by the library instead
    o2 = rk.flash_attn_f16(pad_heads(q, d), pad_heads(k, d), vt, s, s, d, h, h, d ** -0.5, 0.0, mode, dv=dvp)
    assert (o2[:, :, d:] == 0).all()
    check(orc, o2[:, :, :d].transpose(1, 0, 2).reshape(s, h * d).astype(np.float32), got)


@pytest.mark.parametrize("hd,dv", [(32, 16), (64, 48), (96, 112), (160, 144), (192, 192), (224, 64)])
def test_flash_attn_head_dims_of_the_reference_contract(rk, orc, hd, dv):
    """`check_flash` accepts any head_dim % 32 and dv % 16 (attn/mod.rs:1443):
    widths between the kernel's run on the next kernel width, zero-padded.
    Checked against the oracle on operands zero-padded to a common width
    (zero q/k columns leave the scores, zero V columns give zero outputs)."""
    s, h, kv = 150, 4, 2
    note(f"flash_attn head_dim {hd} dv {dv}")
    r = np.random.default_rng(hd * 7 + dv)
    w = max(hd, dv)
    q = np.zeros((h, s, w), np.float16)
    k = np.zeros((kv, s, w), np.float16)
    v = np.zeros((kv, s, w), np.float16)
    q[:, :, :hd] = r.standard_normal((h, s, hd))
    k[:, :, :hd] = r.standard_normal((kv, s, hd))
    v[:, :, :dv] = r.standard_normal((kv, s, dv))
    vt = np.ascontiguousarray(v[:, :, :dv].transpose(0, 2, 1))  # [kv][dv][s]
    for mode in (0, 1):
        o = rk.flash_attn_f16(np.ascontiguousarray(q[:, :, :hd]), np.ascontiguousarray(k[:, :, :hd]), vt, s, s,
                              hd, h, kv, hd ** -0.5, 0.0, mode, dv=dv)
        assert o.shape == (h, s, dv)
        got = o.transpose(1, 0, 2).reshape(s, h * dv).astype(np.float32)
        tok = lambda x: x.transpose(1, 0, 2).reshape(s, -1)  # [heads][s][w] → [s, heads·w]
        ref = orc.attention_ref(tok(q), tok(k), tok(v), h, kv, w, hd ** -0.5, 0.0, mode)
        ref = ref.reshape(s, h, w)[:, :, :dv].reshape(s, h * dv)
        check(orc, got, ref)


@pytest.mark.parametrize("d", [160, 192, 224])
def test_token_major_head_dims_run_padded(rk, orc, d):
    """rk_attention_dev and rk_attention take the head dims of the reference's
    contract between the kernel widths (head_dim % 32 above 128) and run them
    zero-padded to 256; the no-allocation entry and token strides wider than
    the packed rows refuse them."""
    note(f"token-major head dim {d} (padded to 256)")
    r = np.random.default_rng(d)
    n, h, kv = 130, 4, 2
    q = r.standard_normal((n, h * d)).astype(np.float16)
    k = r.standard_normal((n, kv * d)).astype(np.float16)
    v = r.standard_normal((n, kv * d)).astype(np.float16)
    for mode in (0, 1):
        got = attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, mode=mode)
        check(orc, got, orc.attention_ref(q, k, v, h, kv, d, d ** -0.5, 0.0, mode))
    host = rk.attention(q[None].astype(np.float32), k[None].astype(np.float32), v[None].astype(np.float32), h, kv, d,
                        d ** -0.5, is_causal=True)
    check(orc, np.asarray(host, np.float32).reshape(n, h * d), orc.attention_ref(q, k, v, h, kv, d, d ** -0.5, 0.0, 1))
    lib = rk.lib()
    bufs = [rk.DeviceBuffer.from_array(np.ascontiguousarray(a).view(np.uint16)) for a in (q, k, v)]
    out = rk.DeviceBuffer(n * h * d * 2)
    assert lib.rk_attention_dev_noalloc(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, n, n, h, kv, d, 0.1, 0.0, 0, -1, 0, 0,
                                        out.ptr, None) == rk.RK_E_UNSUPPORTED
    wide = rk.DeviceBuffer(n * (h * d + 8) * 2)
    assert lib.rk_attention_strided_dev(wide.ptr, h * d + 8, bufs[1].ptr, kv * d, bufs[2].ptr, kv * d, n, n, h, kv,
                                        d, 0.1, 0.0, 0, -1, 0, 0, out.ptr, h * d, None) == rk.RK_E_UNSUPPORTED


def test_attention_rejects_bad_shapes(rk):
    note("attention errors")
    lib = rk.lib()
    assert lib.rk_attention(None, None, None, 4, 4, 6, 4, 128, 1.0, 0.0, 0, -1, 0, 0, None) == rk.RK_E_SHAPE
    assert lib.rk_attention(None, None, None, 4, 4, 4, 4, 40, 1.0, 0.0, 0, -1, 0, 0, None) == rk.RK_E_UNSUPPORTED


def test_attention_is_deterministic(rk, orc):
    # Same inputs, same bits: every sum has a fixed order (a split query tile's
    # two halves are merged in split order, whichever finishes second).
    c = synth.MOE
    s, h, kv, d = c["s"], c["attn_heads"], c["attn_kv"], c["attn_d"]
    note(f"determinism S={s} H={h} KV={kv}")
    seeds = synth.SEEDS["moe"]
    q = synth.normal_f16(seeds[6], (s, h * d))
    k = synth.normal_f16(seeds[7], (s, kv * d))
    v = synth.normal_f16(seeds[8], (s, kv * d))
    a = attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, mode=1)
    b = attn_dev(rk, q, k, v, h, kv, d, d ** -0.5, mode=1)
    assert (a == b).all()
    check(orc, a, orc.attention_flex(q, k, v, h, kv, d, d ** -0.5, 0.0, 1))


@pytest.mark.parametrize("mode", [0, 1])
def test_head_padding_invariance(rk, orc, mode):
    """Zero-padding the head dim 72 → 80 / 96 (the reference's padded-layout test,
    src/clef/vision/tests.rs:411-473): the padded output columns are exactly zero and the
    rest is the plain attention within the reference's max-abs bound 2e-3 of the f64 model.
    The scale stays 72^-0.5."""
    s, h, d = 157, 4, 72
    r = np.random.default_rng(72 + mode)
    q = r.standard_normal((s, h * d)).astype(np.float16)
    k = r.standard_normal((s, h * d)).astype(np.float16)
    v = r.standard_normal((s, h * d)).astype(np.float16)
    want = orc.attention_ref(q, k, v, h, h, d, d ** -0.5, 0.0, mode)
    for dp in (80, 96):
        note(f"head padding 72 -> {dp}, mode {mode}")

        def pad(x):
            out = np.zeros((s, h, dp), np.float16)
            out[:, :, :d] = x.reshape(s, h, d)
            return out.reshape(s, h * dp)

        got = attn_dev(rk, pad(q), pad(k), pad(v), h, h, dp, d ** -0.5, mode=mode).reshape(s, h, dp)
        assert (got[:, :, d:] == 0).all()
        assert np.abs(got[:, :, :d].reshape(s, h * d) - want).max() < 2e-3
