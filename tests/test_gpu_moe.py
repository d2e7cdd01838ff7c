"""GPU parity of the MoE expert pipeline (K4: grouped W8A8 GEMMs over per-expert
token lists, silu·up, down, combine) against the oracle's W8A8 emulation."""
import sys

import numpy as np
import pytest

from burn_rocket import synth

pytestmark = pytest.mark.gpu
COS_MIN, REL_MAX = 0.9999, 1e-2


def note(msg):
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def make_experts(orc, seed, E, H, I):
    """Q8_0 expert stack: codes/scales for the oracle and GGUF blocks for the pack."""
    gq = np.empty((E, I, H), np.int8)
    uq = np.empty((E, I, H), np.int8)
    dq = np.empty((E, H, I), np.int8)
    gd = np.empty((E, I, H // 32), np.uint16)
    ud = np.empty((E, I, H // 32), np.uint16)
    dd = np.empty((E, H, I // 32), np.uint16)
    for e in range(E):
        gq[e], gd[e] = orc.q8_0_quantize(synth.normal_f32(seed + 3 * e, (I, H), 0.02))
        uq[e], ud[e] = orc.q8_0_quantize(synth.normal_f32(seed + 3 * e + 1, (I, H), 0.02))
        dq[e], dd[e] = orc.q8_0_quantize(synth.normal_f32(seed + 3 * e + 2, (H, I), 0.02))
    blocks = [orc.q8_0_blocks(q.reshape(-1, q.shape[-1]), d.reshape(-1, d.shape[-1]))
              for q, d in ((gq, gd), (uq, ud), (dq, dd))]
    f = lambda d: d.view(np.float16).astype(np.float32)
    return dict(gq=gq, gs=f(gd), uq=uq, us=f(ud), dq=dq, ds=f(dd), blocks=blocks)


def run_moe(rk, wid, x, ids, wts):
    s, H = x.shape
    dx = rk.DeviceBuffer.from_array(x)
    dy = rk.DeviceBuffer(x.nbytes)
    ids = np.ascontiguousarray(ids, np.uint32)
    wts = np.ascontiguousarray(wts, np.float32)
    rc = rk.lib().rk_moe_experts_dev(int(wid), dx.ptr, s, ids.shape[1], ids.ctypes.data, wts.ctypes.data, dy.ptr,
                                     None)
    assert rc == 0, rk.lib().rk_last_error()
    rk.synchronize()
    return dy.download((s, H), np.float32)


@pytest.mark.parametrize("S,H,I,E,K", [(256, 512, 256, 16, 4), (300, 256, 128, 8, 8), (5, 128, 64, 4, 2)])
def test_moe_pipeline_matches_emulation(rk, orc, S, H, I, E, K):
    note(f"MoE S={S} H={H} I={I} E={E} top{K}")
    r = np.random.default_rng(S + E)
    ex = make_experts(orc, 700 + E, E, H, I)
    wid = rk.pack_moe_q8_0(*ex["blocks"], E, H, I)
    x = r.standard_normal((S, H)).astype(np.float32)
    ids, wts = rk.moe_route(r.standard_normal((S, E)).astype(np.float32), K)
    got = run_moe(rk, wid, x, ids, wts)
    ref = orc.moe_experts(x, ids, wts, ex["gq"], ex["gs"], ex["uq"], ex["us"], ex["dq"], ex["ds"])
    assert np.isfinite(got).all()
    cos, rel = orc.cosine(got, ref), orc.max_rel(got, ref)
    assert cos >= COS_MIN and rel <= REL_MAX, (cos, rel)


def test_moe_skewed_routing_over_128_rows_per_expert(rk, orc):
    # Every token picks experts 0 and 1: 600 rows per expert span several tiles.
    note("MoE skewed routing")
    S, H, I, E = 600, 128, 64, 4
    ex = make_experts(orc, 900, E, H, I)
    wid = rk.pack_moe_q8_0(*ex["blocks"], E, H, I)
    r = np.random.default_rng(1)
    x = r.standard_normal((S, H)).astype(np.float32)
    ids = np.tile(np.array([[1, 0]], np.uint32), (S, 1))
    wts = np.tile(np.array([[0.7, 0.3]], np.float32), (S, 1))
    got = run_moe(rk, wid, x, ids, wts)
    ref = orc.moe_experts(x, ids, wts, ex["gq"], ex["gs"], ex["uq"], ex["us"], ex["dq"], ex["ds"])
    assert orc.cosine(got, ref) >= COS_MIN and orc.max_rel(got, ref) <= REL_MAX


def test_moe_config5_subset_of_experts(rk, orc):
    # Config-5 expert shapes (hidden 2048, inter 768, top-8 of 128 logits) on
    # 16 resident experts, with the router over those 16.
    c = synth.MOE
    S, H, I, E, K = 512, c["hidden"], c["inter"], 16, c["top_k"]
    note(f"MoE config5 shapes S={S} H={H} I={I} E={E} top{K}")
    ex = make_experts(orc, synth.SEEDS["moe"][2], E, H, I)
    wid = rk.pack_moe_q8_0(*ex["blocks"], E, H, I)
    x = synth.normal_f32(synth.SEEDS["moe"][0], (S, H))
    ids, wts = rk.moe_route(synth.normal_f32(synth.SEEDS["moe"][1], (S, E)), K)
    got = run_moe(rk, wid, x, ids, wts)
    ref = orc.moe_experts(x, ids, wts, ex["gq"], ex["gs"], ex["uq"], ex["us"], ex["dq"], ex["ds"])
    assert orc.cosine(got, ref) >= COS_MIN and orc.max_rel(got, ref) <= REL_MAX
