"""rk_attention_dev_noalloc, the attention entry point that allocates nothing
(its V-transposed operand lives in a static device array), against the
allocating rk_attention_dev on the same inputs, and against the oracle."""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
COS_MIN, REL_MAX = 0.9999, 1e-2


def note(msg):
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def _call(rk, name, bufs, s, h, kv, d, mode, out):
    lib = rk.lib()
    rc = getattr(lib, name)(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, s, s, h, kv, d, d ** -0.5, 0.0, mode, -1, 0,
                            0, out.ptr, None)
    assert rc == 0, lib.rk_last_error()
    rk.synchronize()
    return out.download((s, h * d), np.uint16).view(np.float16).astype(np.float32)


def test_noalloc_attention_equals_rk_attention_dev(rk, orc, monkeypatch):
    # Two calls in a row, the second smaller: the causal Qwen3 shape, then a
    # bidirectional 72-wide one. The static array keeps the first call's Vᵀ;
    # the second call must not see any of it. The no-allocation entry never
    # splits a query tile's keys between workgroups (that takes a workspace),
    # so it equals rk_attention_dev bit for bit with the split off
    # (RK_ATTN_SPLIT=1), and within the parity gate with the default, which
    # splits the small second grid.
    rk.clear_scratch()
    for i, (s, h, kv, d, mode) in enumerate(((3633, 16, 8, 128, 1), (700, 8, 2, 72, 0))):
        note(f"noalloc attention S={s} H={h} KV={kv} D={d} mode={mode}")
        r = np.random.default_rng(90 + i)
        q = r.standard_normal((s, h * d)).astype(np.float16)
        k = r.standard_normal((s, kv * d)).astype(np.float16)
        v = r.standard_normal((s, kv * d)).astype(np.float16)
        bufs = [rk.DeviceBuffer.from_array(t.view(np.uint16)) for t in (q, k, v)]
        out = rk.DeviceBuffer(s * h * d * 2)
        held = rk.mem_stats().scratch_bytes
        got = _call(rk, "rk_attention_dev_noalloc", bufs, s, h, kv, d, mode, out)
        assert rk.mem_stats().scratch_bytes == held  # no library scratch taken
        monkeypatch.setenv("RK_ATTN_SPLIT", "1")
        want = _call(rk, "rk_attention_dev", bufs, s, h, kv, d, mode, rk.DeviceBuffer(s * h * d * 2))
        assert (got == want).all()  # the same kernels on the same operands
        monkeypatch.delenv("RK_ATTN_SPLIT")
        dflt = _call(rk, "rk_attention_dev", bufs, s, h, kv, d, mode, rk.DeviceBuffer(s * h * d * 2))
        assert orc.cosine(got, dflt) >= COS_MIN and orc.max_rel(got, dflt) <= REL_MAX
        for a, b in ((0, 40), (s // 2, s // 2 + 40), (s - 40, s)):
            ref = orc.attention_ref(q[a:b], k, v, h, kv, d, d ** -0.5, 0.0, mode, -1, a, 0)
            assert orc.cosine(got[a:b], ref) >= COS_MIN and orc.max_rel(got[a:b], ref) <= REL_MAX


def test_noalloc_attention_rejects_shapes_beyond_its_scratch(rk):
    # 8 kv heads × 128 × round_up(16385, 64) keys × 2 bytes is just above 32 MiB:
    # refused on the host before any work is queued.
    note("noalloc attention size limit")
    lib = rk.lib()
    h, kv, d = 8, 8, 128
    for n_kv, ok in ((16384, True), (16385, False)):
        need = kv * d * ((n_kv + 63) // 64 * 64) * 2
        assert (need <= rk.NOALLOC_SCRATCH_BYTES) == ok
    n_q, n_kv = 4, 16385
    bufs = [rk.DeviceBuffer(n_q * h * d * 2), rk.DeviceBuffer(n_kv * kv * d * 2), rk.DeviceBuffer(n_kv * kv * d * 2)]
    for b in bufs:
        b.zero()
    out = rk.DeviceBuffer(n_q * h * d * 2)
    rc = lib.rk_attention_dev_noalloc(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, n_q, n_kv, h, kv, d, 0.1, 0.0, 0, -1,
                                      0, 0, out.ptr, None)
    assert rc == rk.RK_E_NOMEM
    assert b"static scratch" in lib.rk_last_error()


def test_noalloc_attention_refuses_the_padded_head_dims(rk):
    # rk_attention_dev runs head dims 160, 192 and 224 zero-padded to 256 in
    # scratch; the no-allocation entry has no scratch for that and refuses them.
    note("noalloc attention padded head dims")
    lib = rk.lib()
    n, h, kv = 64, 2, 1
    for d in (160, 192, 224):
        q = rk.DeviceBuffer(n * h * d * 2)
        k = rk.DeviceBuffer(n * kv * d * 2)
        out = rk.DeviceBuffer(n * h * d * 2)
        q.zero()
        k.zero()
        rc = lib.rk_attention_dev_noalloc(q.ptr, k.ptr, k.ptr, n, n, h, kv, d, 0.1, 0.0, 0, -1, 0, 0, out.ptr, None)
        assert rc == rk.RK_E_UNSUPPORTED, d
        # the allocating entry accepts the same call
        assert lib.rk_attention_dev(q.ptr, k.ptr, k.ptr, n, n, h, kv, d, 0.1, 0.0, 0, -1, 0, 0, out.ptr, None) == 0
    rk.synchronize()
