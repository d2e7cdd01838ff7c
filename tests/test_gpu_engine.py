"""GPU tests of the engine state around the ops: scratch shared by calls on
different streams, the stats counters (`burn_rocket::stats`, ext.rs:165-200)
and scratch trimming (`trim_scratch_to` / `clear_scratch`, ext.rs:256-308)."""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
COS_MIN, REL_MAX = 0.9999, 1e-2


def note(msg):
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def _qkv(seed, s, h, kv, d):
    r = np.random.default_rng(seed)
    return (r.standard_normal((s, h * d)).astype(np.float16), r.standard_normal((s, kv * d)).astype(np.float16),
            r.standard_normal((s, kv * d)).astype(np.float16))


def _launch(rk, bufs, s, h, kv, d, mode, out, stream):
    lib = rk.lib()
    rc = lib.rk_attention_dev(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, s, s, h, kv, d, d ** -0.5, 0.0, mode, -1,
                              0, 0, out.ptr, ctypes.c_void_p(stream))
    assert rc == 0, lib.rk_last_error()


def _check_rows(orc, got, q, k, v, h, kv, d, mode):
    s = q.shape[0]
    for a, b in ((0, 40), (s // 2, s // 2 + 40), (s - 40, s)):
        ref = orc.attention_flex(q[a:b], k, v, h, kv, d, d ** -0.5, 0.0, mode, -1, a, 0)
        g = got[a:b]
        assert orc.cosine(g, ref) >= COS_MIN and orc.max_rel(g, ref) <= REL_MAX


@pytest.mark.parametrize("second_larger", [False, True])
def test_attention_on_two_streams_back_to_back(rk, orc, second_larger):
    # Both calls rewrite V into the same internal scratch. The second call is
    # issued on another stream right after the first, with no host sync in
    # between; it must wait for the first on the device (smaller second call)
    # or free the buffer only after the first finished (larger second call).
    shapes = [(3633, 16, 8, 128, 1), (700, 8, 2, 64, 0)]
    if second_larger:
        shapes.reverse()
    note(f"two streams: {shapes}")
    s1, s2 = rk.new_stream(), rk.new_stream()
    try:
        runs = []
        for i, (s, h, kv, d, mode) in enumerate(shapes):
            q, k, v = _qkv(40 + i, s, h, kv, d)
            bufs = [rk.DeviceBuffer.from_array(t.view(np.uint16)) for t in (q, k, v)]
            out = rk.DeviceBuffer(s * h * d * 2)
            runs.append((q, k, v, bufs, out, s, h, kv, d, mode))
        for (q, k, v, bufs, out, s, h, kv, d, mode), st in zip(runs, (s1, s2)):
            _launch(rk, bufs, s, h, kv, d, mode, out, st)
        rk.synchronize(s1)
        rk.synchronize(s2)
        for q, k, v, bufs, out, s, h, kv, d, mode in runs:
            got = out.download((s, h * d), np.uint16).view(np.float16).astype(np.float32)
            _check_rows(orc, got, q, k, v, h, kv, d, mode)
    finally:
        rk.synchronize(s1)
        rk.synchronize(s2)
        rk.destroy_stream(s1)
        rk.destroy_stream(s2)


def test_stats_count_host_ops_and_split_their_time(rk, orc):
    note("stats")
    r = np.random.default_rng(11)
    w = (r.standard_normal((256, 512)) * 0.05).astype(np.float32)
    x = r.standard_normal((96, 512)).astype(np.float32)
    wid = rk.pack(w)
    rk.stats_reset()
    s0 = rk.stats()
    assert s0.calls == 0 and s0.convert_s == 0.0 and s0.npu_s == 0.0
    y = rk.matmul(x, wid)
    s1 = rk.stats()
    assert s1.calls == 1 and s1.convert_s > 0.0 and s1.npu_s > 0.0
    ref = orc.gemm_f16(orc.f32_to_f16(x), orc.f32_to_f16(w))
    assert orc.cosine(y, ref) >= COS_MIN
    h, kv, d, n = 4, 2, 64, 50
    q = r.standard_normal((1, n, h * d)).astype(np.float32)
    k = r.standard_normal((1, n, kv * d)).astype(np.float32)
    rk.attention(q, k, k, h, kv, d, d ** -0.5, None, True)
    s2 = rk.stats()
    assert s2.calls == 2 and s2.convert_s > s1.convert_s and s2.npu_s > s1.npu_s
    # a device-buffer call counts but adds no time (it returns before its kernels end)
    a16 = rk.DeviceBuffer.from_array(orc.f32_to_f16(x))
    c16 = rk.DeviceBuffer(96 * 256 * 2)
    assert rk.lib().rk_matmul_f16_dev(int(wid), a16.ptr, 96, 512, c16.ptr, None) == 0
    rk.synchronize()
    s3 = rk.stats()
    assert s3.calls == 3 and s3.convert_s == s2.convert_s and s3.npu_s == s2.npu_s
    rk.stats_reset()
    assert rk.stats().calls == 0


def test_trim_and_clear_scratch(rk, orc):
    note("trim / clear scratch")
    s, h, kv, d = 512, 8, 4, 128
    q, k, v = _qkv(7, s, h, kv, d)
    out = rk.attention(q.astype(np.float32)[None], k.astype(np.float32)[None], v.astype(np.float32)[None],
                       h, kv, d, d ** -0.5, None, True)
    held = rk.mem_stats().scratch_bytes
    assert held > 0
    budget = held // 2
    rk.trim_scratch_to(budget)
    assert rk.mem_stats().scratch_bytes <= budget
    rk.clear_scratch()
    assert rk.mem_stats().scratch_bytes == 0
    # the op still works, and gives the same bits, after its scratch was dropped
    again = rk.attention(q.astype(np.float32)[None], k.astype(np.float32)[None], v.astype(np.float32)[None],
                         h, kv, d, d ** -0.5, None, True)
    assert (again == out).all()
    assert rk.mem_stats().scratch_bytes > 0


def test_moe_plan_run_on_a_caller_stream_then_destroyed(rk, orc):
    # rk_moe_plan_destroy must wait for a run on another stream that reads the
    # plan's device lists before it frees them.
    note("MoE plan on a caller stream")
    E, H, I, S, K = 8, 256, 128, 200, 4
    r = np.random.default_rng(12)
    gate = (r.standard_normal((E, I, H)) * 0.05).astype(np.float32)
    up = (r.standard_normal((E, I, H)) * 0.05).astype(np.float32)
    down = (r.standard_normal((E, H, I)) * 0.05).astype(np.float32)
    wid = rk.pack_moe_f32(gate, up, down)
    x = r.standard_normal((S, H)).astype(np.float32)
    ids, wts = rk.moe_route(r.standard_normal((S, E)).astype(np.float32), K)
    ids, wts = np.ascontiguousarray(ids), np.ascontiguousarray(wts)
    lib = rk.lib()
    ref_y = rk.DeviceBuffer(S * H * 4)
    dx = rk.DeviceBuffer.from_array(x)
    assert lib.rk_moe_experts_dev(int(wid), dx.ptr, S, K, ids.ctypes.data, wts.ctypes.data, ref_y.ptr, None) == 0
    rk.synchronize()
    st = rk.new_stream()
    try:
        plan = ctypes.c_void_p()
        assert lib.rk_moe_plan_create(int(wid), S, K, ids.ctypes.data, wts.ctypes.data, ctypes.byref(plan)) == 0
        dy = rk.DeviceBuffer(S * H * 4)
        assert lib.rk_moe_experts_planned_dev(int(wid), plan, dx.ptr, dy.ptr, ctypes.c_void_p(st)) == 0
        assert lib.rk_moe_plan_destroy(plan) == 0
        rk.synchronize(st)
        assert (dy.download((S, H), np.float32) == ref_y.download((S, H), np.float32)).all()
    finally:
        rk.synchronize(st)
        rk.destroy_stream(st)
