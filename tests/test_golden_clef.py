"""The oracle's MoE router and expert combine against the reference's torch
golden vectors (CPU).

The reference pins its Clef decoder layer with a tiny synthetic model whose
weights are a closed formula and whose expected outputs were produced by a
torch manual layer (src/clef/model/tests.rs:79-112 with the vectors of
src/clef/model/mini_expected.in, extracted to tests/golden/clef_mini_expected.json
by tests/golden/make_clef_mini.py). This test restates that layer in numpy
(src/clef/model.rs:330-386 RoPE, 407-422 RMSNorm, 425-460 causal GQA attention,
526-621 layer with router and MoE) around two oracle functions:

* orc.route must reproduce the golden router ids exactly and the weights to
  1e-5 (the reference test's bounds), from logits the numpy layer computes;
* the layer output, with the expert FFN and the ascending-expert-id combine,
  must match the golden hidden states to 2e-6 of the peak (the reference's
  bound); orc.moe_experts, the W8A8 (Q8_0 weights, int8 activations per
  32-value group) restatement of that FFN + combine, must stay within the
  quantization error of it (cosine >= 0.9999 on the layer output).
"""
import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "clef_mini_expected.json")))

H, LAYERS, NH, NKV, D, E, TOPK, I, EPS, THETA = 64, 2, 4, 2, 16, 4, 2, 32, 1e-6, 1e6
S = 5


def val(n, salt, scale):
    return (np.sin(np.arange(n) * 0.37 + salt) * scale).astype(np.float32)


def one_plus(n, salt, scale):
    return (np.float32(1.0) + val(n, salt, scale)).astype(np.float32)


def mini_layer(l):
    s = 10.0 * l
    w = dict(input_norm=one_plus(H, s + 1, 0.1), post_norm=one_plus(H, s + 2, 0.1),
             q=val(NH * D * H, s + 3, 0.3).reshape(NH * D, H), k=val(NKV * D * H, s + 4, 0.3).reshape(NKV * D, H),
             v=val(NKV * D * H, s + 5, 0.3).reshape(NKV * D, H), o=val(H * NH * D, s + 6, 0.3).reshape(H, NH * D),
             q_norm=one_plus(D, s + 7, 0.1), k_norm=one_plus(D, s + 8, 0.1),
             router=val(E * H, s + 9, 0.5).reshape(E, H))
    ex = [(val(I * H, s + 20 + e, 0.3).reshape(I, H), val(I * H, s + 30 + e, 0.3).reshape(I, H),
           val(H * I, s + 40 + e, 0.3).reshape(H, I)) for e in range(E)]
    return w, ex


def mm(a, b):  # a [m, k] · b[n, k]ᵀ in f32 (accumulated in f64)
    return (a.astype(np.float64) @ b.astype(np.float64).T).astype(np.float32)


def rms_norm(x, w):
    ms = (x.astype(np.float64) ** 2).mean(axis=-1, keepdims=True)
    inv = np.float32(1.0) / np.sqrt(ms.astype(np.float32) + np.float32(EPS))
    return (w * (x * inv)).astype(np.float32)


def rope(x, heads):
    half = D // 2
    inv = (1.0 / THETA ** (np.arange(half) * 2 / D)).astype(np.float32)
    ang = (np.arange(S, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    c, s_ = np.cos(ang.astype(np.float64)).astype(np.float32), np.sin(ang.astype(np.float64)).astype(np.float32)
    x = x.reshape(S, heads, D).copy()
    a, b = x[..., :half].copy(), x[..., half:].copy()
    x[..., :half] = a * c[:, None, :] - b * s_[:, None, :]
    x[..., half:] = b * c[:, None, :] + a * s_[:, None, :]
    return x.reshape(S, heads * D)


def attention(q, k, v):
    rep, scale = NH // NKV, np.float32(1.0 / np.sqrt(np.float32(D)))
    ctx = np.zeros((S, NH * D), np.float32)
    for i in range(S):
        for h in range(NH):
            g = h // rep
            qi = q[i, h * D:(h + 1) * D].astype(np.float64)
            sc = np.array([qi @ k[j, g * D:(g + 1) * D] for j in range(i + 1)], np.float32) * scale
            p = np.exp((sc - sc.max()).astype(np.float64)).astype(np.float32)
            p = p / p.sum(dtype=np.float32)
            ctx[i, h * D:(h + 1) * D] = (p.astype(np.float64) @ v[:i + 1, g * D:(g + 1) * D]).astype(np.float32)
    return ctx


def silu(x):
    return (x / (np.float32(1.0) + np.exp(-x.astype(np.float64)).astype(np.float32))).astype(np.float32)


def layer(orc, l, x):
    w, ex = mini_layer(l)
    n = rms_norm(x, w["input_norm"])
    q = rms_norm(mm(n, w["q"]).reshape(S, NH, D), w["q_norm"]).reshape(S, NH * D)
    k = rms_norm(mm(n, w["k"]).reshape(S, NKV, D), w["k_norm"]).reshape(S, NKV * D)
    v = mm(n, w["v"])
    hid = (x + mm(attention(rope(q, NH), rope(k, NKV), v), w["o"])).astype(np.float32)
    n2 = rms_norm(hid, w["post_norm"])
    ids, wts = orc.route(mm(n2, w["router"]), TOPK, True)
    y = hid.copy()
    for e in range(E):  # ascending expert id, rows in token order
        for t in range(S):
            for slot in range(TOPK):
                if ids[t, slot] == e:
                    g, u, dn = ex[e]
                    a = silu(mm(n2[t:t + 1], g)) * mm(n2[t:t + 1], u)
                    y[t] += mm(a.astype(np.float32), dn)[0] * wts[t, slot]
    return y, ids, wts, hid, n2, ex


def test_router_and_layer_match_the_torch_goldens(orc):
    x = val(S * H, 99.0, 1.0).reshape(S, H)
    for l in range(LAYERS):
        y, ids, wts, _, _, _ = layer(orc, l, x)
        assert ids.reshape(-1).tolist() == GOLD[f"IDS_L{l}"], f"layer {l} router ids"
        assert np.abs(wts.reshape(-1) - np.array(GOLD[f"WTS_L{l}"], np.float32)).max() < 1e-5
        want = np.array(GOLD[f"HIDDEN_L{l}"], np.float32).reshape(S, H)
        peak = np.abs(want).max()
        assert np.abs(y - want).max() / peak < 2e-6, (l, np.abs(y - want).max() / peak)
        x = y


def test_w8a8_expert_combine_stays_within_quantization_error_of_the_goldens(orc):
    x = val(S * H, 99.0, 1.0).reshape(S, H)
    for l in range(LAYERS):
        _, ids, wts, hid, n2, ex = layer(orc, l, x)
        q = [orc.q8_0_quantize(np.stack([ex[e][p] for e in range(E)]).reshape(-1, ex[0][p].shape[1]))
             for p in range(3)]
        f = lambda d: d.view(np.float16).astype(np.float32)
        gq, gs = q[0][0].reshape(E, I, H), f(q[0][1]).reshape(E, I, H // 32)
        uq, us = q[1][0].reshape(E, I, H), f(q[1][1]).reshape(E, I, H // 32)
        dq, ds = q[2][0].reshape(E, H, I), f(q[2][1]).reshape(E, H, I // 32)
        y = hid + orc.moe_experts(n2, ids, wts, gq, gs, uq, us, dq, ds)
        want = np.array(GOLD[f"HIDDEN_L{l}"], np.float32).reshape(S, H)
        assert orc.cosine(y, want) >= 0.9999, (l, orc.cosine(y, want))
        x = want
