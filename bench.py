#!/usr/bin/env python3
"""Benchmark of the burn-rocket MI355X op surface on one GPU.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extras] [--no-cpu-baseline]

A step is one pass of the headline workload: the Q8_0/W8A8 MLP GEMMs at
M=3633 tokens — up-projection K=1024→N=3072 and down-projection K=3072→N=1024
— on per-token int8 activations and Q8_0 weights that are resident in HBM
when the timed region starts. `value` is int8 tera-ops per second over the K
timed steps (2·M·K·N per GEMM), measured with HIP events on the library
stream around the whole timed region. `roofline` is the up-projection
kernel's average launch time (K back-to-back launches between two events on
the same stream, right after the timed region) against the MI355X dense int8
MFMA peak. `extras` times the other four workloads the same way, before the
headline (the card's clocks then have settled when its steps are timed), except
the host-buffer pass, which runs after it; `cpu_baseline` times the oracle's C
restatement of the reference's W8A8 path
on the host cores (all of them, and one core) over a bounded sample; every
`extras` entry carries its own `cpu_baseline` of the same kind.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "burn-rocket_amd"))

import numpy as np  # noqa: E402

import burn_rocket as rk  # noqa: E402
from burn_rocket import synth  # noqa: E402

METRIC = "GEMM & GQA-attn TFLOP/s + % MFMA peak on 1 MI355X vs host-CPU Burn path"
PEAK_FP16 = 2516.6  # TFLOP/s dense
PEAK_INT8 = 5033.2  # TOP/s dense
PEAK_HBM = 8000.0   # GB/s
# VALU lane-operations per second: 256 CUs × 4 SIMDs × 16 lanes × 2.4 GHz.
PEAK_VALU = 256 * 4 * 16 * 2.4e9
# TOP/s at which a W8A8 GEMM with one scale per 32-value block saturates the
# VALU on its fold alone (2 operations per output element and block, each
# worth 64 int8 operations of the product): 64 / 2 · PEAK_VALU.
VALU_FOLD_CEILING = 64 / 2 * PEAK_VALU / 1e12


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def dev(a):
    return rk.DeviceBuffer.from_array(np.ascontiguousarray(a))


def call(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: {rk.lib().rk_last_error().decode()}")


def time_launches(fn, iters, warmup=3, warm_s=0.03):
    """Average ms per call of fn() measured with events on the library stream.
    Untimed calls run first for at least `warmup` calls and `warm_s` seconds: after
    host-side set-up the card's clocks need ~10 ms of work to come back up (a
    30B-A3B expert layer measures 300 µs cold against 256 µs warm)."""
    t0, n = time.perf_counter(), 0
    while n < warmup or time.perf_counter() - t0 < warm_s:
        fn()
        n += 1
        if n % 8 == 0:
            rk.synchronize()
    rk.synchronize()
    e0, e1 = rk.Event(), rk.Event()
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    rk.synchronize()
    return e0.elapsed_ms(e1) / iters


# ------------------------------------------------------------ config 2 ----
def setup_w8a8():
    c = synth.W8A8
    s1, s2, s3 = synth.SEEDS["w8a8"]
    m, h, i = c["m"], c["hidden"], c["inter"]
    lib = rk.lib()
    layers = []
    for name, k, n, sx, sw in (("up", h, i, s1, s2), ("down", i, h, s1 + 1000, s3)):
        x = synth.normal_f32(sx, (m, k))
        w = synth.normal_f32(sw, (n, k), 0.02)
        wid = rk.pack_q8_0_f32(w)
        dx = dev(x)
        dq, ds = rk.DeviceBuffer(m * k), rk.DeviceBuffer(m * 4)
        call(lib.rk_quantize_rows_dev(dx.ptr, m, k, k, dq.ptr, ds.ptr, None), "quantize")
        dc = rk.DeviceBuffer(m * n * 4)
        layers.append(dict(name=name, m=m, k=k, n=n, wid=wid, dx=dx, dq=dq, ds=ds, dc=dc,
                           sha_x=synth.sha256(x), sha_w=synth.sha256(w)))
    rk.synchronize()
    return layers


def gemm_w8a8(L):
    call(rk.lib().rk_matmul_w8a8_dev(int(L["wid"]), L["dq"].ptr, L["ds"].ptr, L["k"], L["m"], L["k"],
                                     L["dc"].ptr, None), "w8a8")


def run_headline(layers, steps, warmup):
    """Timed steps (up + down), events only around the whole region; then the
    up-projection kernel alone, `steps` back-to-back launches between two
    events on the same stream, for its average launch duration."""
    up, down = layers
    for _ in range(warmup):
        gemm_w8a8(up)
        gemm_w8a8(down)
    rk.synchronize()
    e0, e1 = rk.Event(), rk.Event()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        gemm_w8a8(up)
        gemm_w8a8(down)
    e1.record()
    rk.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1) / steps
    up_ms = time_launches(lambda: gemm_w8a8(up), steps, warmup=2)
    return ms, up_ms, wall


COPY_PROBE_BYTES = 256 << 20
TRAFFIC_LAUNCHES = 10


def traffic_probe(layers, launches):
    """Launches for the rocprofv3 --pmc byte counters: a plain device copy of
    COPY_PROBE_BYTES (its FETCH_SIZE / WRITE_SIZE calibrate the counters), then
    the up- and down-projection kernels `launches` times each."""
    lib = rk.lib()
    src, dst = rk.DeviceBuffer(COPY_PROBE_BYTES), rk.DeviceBuffer(COPY_PROBE_BYTES)
    call(lib.rk_memset_dev(src.ptr, 1, COPY_PROBE_BYTES), "memset")
    for _ in range(launches):
        call(lib.rk_memcpy_dtod(dst.ptr, src.ptr, COPY_PROBE_BYTES, None), "copy")
    rk.synchronize()
    for L in layers:
        for _ in range(launches):
            gemm_w8a8(L)
        rk.synchronize()
    log(f"traffic probe: {launches} copies of {COPY_PROBE_BYTES} B, {launches} launches per projection")


def probe_all(launches):
    """A few launches of every workload's kernels (for rocprofv3 --pmc runs,
    which serialise and count each dispatch): the W8A8 pair (per-token and
    group-32 activations), the fp16 GEMMs, the four attentions and the MoE
    experts."""
    layers = setup_w8a8()
    lib = rk.lib()
    for L in layers:
        for _ in range(launches):
            gemm_w8a8(L)
    # the same pair in the reference's group-32 activation form
    for L in layers:
        m, k = L["m"], L["k"]
        q32, s32 = rk.DeviceBuffer(m * k), rk.DeviceBuffer(m * (k // 32) * 4)
        call(lib.rk_quantize_rows_dev(L["dx"].ptr, m, k, 32, q32.ptr, s32.ptr, None), "quantize g32")
        for _ in range(launches):
            call(lib.rk_matmul_w8a8_dev(int(L["wid"]), q32.ptr, s32.ptr, 32, m, k, L["dc"].ptr, None), "w8a8 g32")
    rk.synchronize()
    for (m, k, n) in ((512, 1024, 3072), (2394, 1152, 3456), (2394, 1152, 1152), (2394, 1152, 4304),
                      (2394, 4304, 1152)):
        a = synth.normal_f16(11, (m, k))
        b = synth.normal_f16(12, (n, k), 0.02)
        wid, da, dc = rk.pack(b), dev(a.view(np.uint16)), rk.DeviceBuffer(m * n * 2)
        for _ in range(launches):
            call(lib.rk_matmul_f16_dev(int(wid), da.ptr, m, k, dc.ptr, None), "f16")
    rk.synchronize()
    for (s, h, kv, d, causal, seeds) in ((synth.GQA_CAUSAL["s"], 16, 8, 128, True, synth.SEEDS["gqa"]),
                                         (synth.VISION["s"], 16, 16, 72, False, synth.SEEDS["vision"][6:9]),
                                         (synth.MOE["s"], 32, 4, 128, True, synth.SEEDS["moe"][6:9])):
        time_attention(s, h, kv, d, causal, seeds, launches)
    extra_gemma_attention(launches)
    extra_moe(launches)
    rk.synchronize()
    log(f"probe-all: {launches} launches of each workload")


def pmc_summary(paths):
    """Per-kernel HBM bytes per launch from rocprofv3 --pmc CSVs (FETCH_SIZE
    and WRITE_SIZE in KiB per dispatch), each counter scaled by what it reads
    for the probe copy of COPY_PROBE_BYTES. Writes profiles/traffic.json and
    prints a markdown table."""
    import csv
    vals = {}
    for path in paths:
        rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Dispatch_Id"]))
        gemm = 0
        for row in rows:
            name = row["Kernel_Name"]
            if "gemm_i8" in name:
                # traffic_probe launches the up-projection `launches` times, then the down-projection
                name = ("[up] " if gemm < TRAFFIC_LAUNCHES else "[down] ") + name
                gemm += 1
            key = (name, int(row["Grid_Size"]))
            vals.setdefault(row["Counter_Name"], {}).setdefault(key, []).append(float(row["Counter_Value"]))
    copy_kib = COPY_PROBE_BYTES / 1024.0
    factor = {}
    for ctr, per in vals.items():
        copies = [v for (name, _), vs in per.items() if "copyBuffer" in name for v in vs]
        factor[ctr] = (sum(copies) / len(copies)) / copy_kib if copies else 1.0
    m, h, i = synth.W8A8["m"], synth.W8A8["hidden"], synth.W8A8["inter"]
    alg = {"w8a8_up": m * h + i * h + 4 * i * h // 32 + 4 * m + 4 * m * i,
           "w8a8_down": m * i + h * i + 4 * h * i // 32 + 4 * m + 4 * m * h}
    out, lines = {}, ["| kernel | grid | FETCH KiB | WRITE KiB | bytes/launch (calibrated) | algorithmic bytes |",
                      "|---|---|---|---|---|---|"]
    keys = sorted({k for per in vals.values() for k in per})
    for name, grid in keys:
        f = vals.get("FETCH_SIZE", {}).get((name, grid), [0.0])
        w = vals.get("WRITE_SIZE", {}).get((name, grid), [0.0])
        fk, wk = sum(f) / len(f), sum(w) / len(w)
        bytes_ = 1024.0 * (fk / factor.get("FETCH_SIZE", 1.0) + wk / factor.get("WRITE_SIZE", 1.0))
        tag = None
        if name.startswith("[up]") or name.startswith("[down]"):
            tag = "w8a8_up" if name.startswith("[up]") else "w8a8_down"
            out[tag] = {"kernel": name[:120], "grid": grid, "fetch_kib": fk, "write_kib": wk,
                        "bytes_per_launch": round(bytes_), "algorithmic_bytes": alg[tag]}
        lines.append(f"| `{name[:80]}` | {grid} | {fk:.0f} | {wk:.0f} | {bytes_ / 1e6:.2f} MB | "
                     f"{alg[tag] / 1e6 if tag else float('nan'):.2f} MB |")
    out["calibration"] = {"copy_bytes": COPY_PROBE_BYTES, "fetch_factor": factor.get("FETCH_SIZE"),
                          "write_factor": factor.get("WRITE_SIZE")}
    with open(os.path.join(ROOT, "profiles", "traffic.json"), "w") as fh:
        json.dump(out, fh, indent=1)
    print("\n".join(lines))
    print(f"\ncalibration: FETCH_SIZE reads {factor.get('FETCH_SIZE', 1.0):.4f}x and WRITE_SIZE "
          f"{factor.get('WRITE_SIZE', 1.0):.4f}x the bytes of a {COPY_PROBE_BYTES >> 20} MiB device copy")


def load_traffic(kernel_key):
    """HBM bytes per launch of a kernel from the committed rocprofv3 --pmc summary."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    try:
        return json.load(open(path)).get(kernel_key, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


# -------------------------------------------------------------- extras ----
def extra_gemm_f16(iters):
    c = synth.GEMM_F16
    s1, s2 = synth.SEEDS["gemm_f16"]
    m, k, n = c["m"], c["k"], c["n"]
    a = synth.normal_f16(s1, (m, k))
    b = synth.normal_f16(s2, (n, k), 0.02)
    lib = rk.lib()
    wid = rk.pack(b)
    da, dc = dev(a.view(np.uint16)), rk.DeviceBuffer(m * n * 2)
    ms = time_launches(lambda: call(lib.rk_matmul_f16_dev(int(wid), da.ptr, m, k, dc.ptr, None), "f16"), iters)
    flop = 2.0 * m * n * k
    # Rotating copies of A and B (> 256 MB) so the operands come from HBM, not the MALL.
    reps = 40
    wids = [rk.pack(b) for _ in range(reps)]
    das = [dev(a.view(np.uint16)) for _ in range(reps)]
    state = {"i": 0}

    def rot():
        j = state["i"] % reps
        state["i"] += 1
        call(lib.rk_matmul_f16_dev(int(wids[j]), das[j].ptr, m, k, dc.ptr, None), "f16")

    ms_rot = time_launches(rot, reps * 5)
    return {"shape": f"{m}x{k}x{n}", "ms": ms, "tflops": flop / ms / 1e9, "frac_fp16_peak": flop / ms / 1e9 / PEAK_FP16,
            "ms_rotating": ms_rot, "tflops_rotating": flop / ms_rot / 1e9}


def attn_flops(s_q, s_k, h, d, causal):
    if causal:
        return 2.0 * d * h * s_q * (s_q + 1)  # unmasked (q, k) pairs, QKᵀ and PV
    return 4.0 * s_q * s_k * d * h


def time_attention(s, h, kv, d, causal, seeds, iters):
    q = synth.normal_f16(seeds[0], (s, h * d))
    k = synth.normal_f16(seeds[1], (s, kv * d))
    v = synth.normal_f16(seeds[2], (s, kv * d))
    dq, dk, dv = dev(q.view(np.uint16)), dev(k.view(np.uint16)), dev(v.view(np.uint16))
    do = rk.DeviceBuffer(s * h * d * 2)
    lib = rk.lib()
    mode = 1 if causal else 0
    ms = time_launches(lambda: call(lib.rk_attention_dev(dq.ptr, dk.ptr, dv.ptr, s, s, h, kv, d, d ** -0.5, 0.0,
                                                         mode, -1, 0, 0, do.ptr, None), "attn"), iters)
    fl = attn_flops(s, s, h, d, causal)
    return {"shape": f"S={s} H={h} KV={kv} D={d} {'causal' if causal else 'bidirectional'}", "ms": ms,
            "tflops": fl / ms / 1e9, "frac_fp16_peak": fl / ms / 1e9 / PEAK_FP16}


def band_pairs(s, window):
    """Visible (query, key) pairs of the bidirectional band |t - j| <= window over s tokens."""
    i = np.arange(s, dtype=np.int64)
    return int((np.minimum(s - 1, i + window) - np.maximum(0, i - window) + 1).sum())


def extra_gemma_attention(iters):
    c = synth.GEMMA_TEXT
    s, h, kv, d, w = c["s"], c["n_head"], c["n_kv"], c["d"], c["window"]
    seeds = synth.SEEDS["gemma"]
    q = synth.normal_f16(seeds[0], (s, h * d))
    k = synth.normal_f16(seeds[1], (s, kv * d))
    v = synth.normal_f16(seeds[2], (s, kv * d))
    dq, dk, dv = dev(q.view(np.uint16)), dev(k.view(np.uint16)), dev(v.view(np.uint16))
    do = rk.DeviceBuffer(s * h * d * 2)
    lib = rk.lib()
    out = {}
    for name, mode, window, pairs in (("full", 0, -1, s * s), ("sliding_512", 2, w, band_pairs(s, w))):
        ms = time_launches(lambda: call(lib.rk_attention_dev(dq.ptr, dk.ptr, dv.ptr, s, s, h, kv, d, d ** -0.5, 0.0,
                                                             mode, window, 0, 0, do.ptr, None), "attn"), iters)
        fl = 4.0 * d * h * pairs  # QKᵀ and PV over the visible pairs
        out[name] = {"shape": f"S={s} H={h} KV={kv} D={d} mode={mode} window={window}", "ms": ms,
                     "tflops": fl / ms / 1e9, "frac_fp16_peak": fl / ms / 1e9 / PEAK_FP16}
    return out


def extra_vision(iters):
    c = synth.VISION
    s, hid, h, d, mlp = c["s"], c["hidden"], c["n_head"], c["d"], c["mlp"]
    seeds = synth.SEEDS["vision"]
    lib = rk.lib()
    x = synth.normal_f16(seeds[0], (s, max(hid, mlp)))
    dx = dev(x.view(np.uint16))
    out = {}
    total_ms, total_fl = 0.0, 0.0
    for i, (name, n, k) in enumerate((("qkv", 3 * hid, hid), ("out", hid, hid), ("fc1", mlp, hid), ("fc2", hid, mlp))):
        w = synth.normal_f16(seeds[1 + i], (n, k), 0.02)
        wid = rk.pack(w)
        xa = dev(x[:, :k].copy().view(np.uint16))
        dc = rk.DeviceBuffer(s * n * 2)
        ms = time_launches(lambda: call(lib.rk_matmul_f16_dev(int(wid), xa.ptr, s, k, dc.ptr, None), "f16"), iters)
        fl = 2.0 * s * n * k
        out[name] = {"ms": ms, "tflops": fl / ms / 1e9, "frac_fp16_peak": fl / ms / 1e9 / PEAK_FP16}
        total_ms += ms
        total_fl += fl
    att = time_attention(s, h, h, d, False, seeds[6:9], iters)
    out["attention"] = att
    total_ms += att["ms"]
    total_fl += attn_flops(s, s, h, d, False)
    out["layer"] = {"ms": total_ms, "tflops": total_fl / total_ms / 1e9}
    return out


_MOE_STATE = {}  # the expert weights and routing, for the CPU baseline of the same workload


def extra_moe(iters):
    c = synth.MOE
    S, H, E, K, I = c["s"], c["hidden"], c["experts"], c["top_k"], c["inter"]
    seeds = synth.SEEDS["moe"]
    log("generating MoE expert weights")
    gate = synth.normal_f32(seeds[2], (E, I, H), 0.02)
    up = synth.normal_f32(seeds[3], (E, I, H), 0.02)
    down = synth.normal_f32(seeds[4], (E, H, I), 0.02)
    wid = rk.pack_moe_f32(gate, up, down)
    x = synth.normal_f32(seeds[0], (S, H))
    ids, wts = rk.moe_route(synth.normal_f32(seeds[1], (S, E)), K)
    _MOE_STATE.update(gate=gate, up=up, down=down, x=x, ids=ids, wts=wts)
    lib = rk.lib()
    import ctypes
    plan = ctypes.c_void_p()
    ids_c, wts_c = np.ascontiguousarray(ids), np.ascontiguousarray(wts)
    call(lib.rk_moe_plan_create(int(wid), S, K, ids_c.ctypes.data, wts_c.ctypes.data, ctypes.byref(plan)), "plan")
    dx, dy = dev(x), rk.DeviceBuffer(S * H * 4)
    ms = time_launches(lambda: call(lib.rk_moe_experts_planned_dev(int(wid), plan, dx.ptr, dy.ptr, None), "moe"),
                       iters)
    call(lib.rk_moe_plan_destroy(plan), "plan")
    ops = 2.0 * S * K * (2 * I * H + H * I)
    weight_bytes = E * (2 * I * H + H * I) * 34 / 32  # Q8_0 codes + f16 scales
    act_bytes = 23.1e6
    att = time_attention(S, c["attn_heads"], c["attn_kv"], c["attn_d"], True, seeds[6:9], iters)
    return {"experts": {"ms": ms, "tops": ops / ms / 1e9, "frac_int8_peak": ops / ms / 1e9 / PEAK_INT8,
                        "gbps_algorithmic": (weight_bytes + act_bytes) / ms / 1e6,
                        "frac_hbm": (weight_bytes + act_bytes) / ms / 1e6 / PEAK_HBM},
            "attention": att}


def extra_w8a8_forms(layers, iters):
    """Config 2 in the reference's own W8A8 form (activations quantized per row per
    32-value group, Σ_g (a_s·w_s)·P_g: matmul_i8 + quantize_i8_rows, ext.rs:1017-1029,
    1505-1554), the raw int32 product of the same codes (no scale fold: the pipeline's
    own ceiling at this shape), and the per-token activation quantizer the headline step
    runs before its timed region."""
    lib = rk.lib()
    out = {}
    g_ms, q_ms, r_ms = 0.0, 0.0, 0.0
    for L in layers:
        m, k = L["m"], L["k"]
        q32, s32 = rk.DeviceBuffer(m * k), rk.DeviceBuffer(m * (k // 32) * 4)
        call(lib.rk_quantize_rows_dev(L["dx"].ptr, m, k, 32, q32.ptr, s32.ptr, None), "quantize g32")
        g_ms += time_launches(lambda: call(lib.rk_matmul_w8a8_dev(int(L["wid"]), q32.ptr, s32.ptr, 32, m, k,
                                                                  L["dc"].ptr, None), "w8a8 g32"), iters)
        # raw int32 product (I8Context::matmul, int8.rs:606-640): no scale fold at all
        r_ms += time_launches(lambda: call(lib.rk_matmul_i8_raw_dev(int(L["wid"]), L["dq"].ptr, m, k, L["dc"].ptr,
                                                                    None), "w8a8 raw"), iters)
        q_ms += time_launches(lambda: call(lib.rk_quantize_rows_dev(L["dx"].ptr, m, k, k, L["dq"].ptr, L["ds"].ptr,
                                                                    None), "quantize"), iters)
    m, h, i = synth.W8A8["m"], synth.W8A8["hidden"], synth.W8A8["inter"]
    ops = 2 * 2.0 * m * h * i
    out["group32_pair"] = {"ms": g_ms, "tops": ops / g_ms / 1e9, "frac_int8_peak": ops / g_ms / 1e9 / PEAK_INT8}
    out["raw_int32_pair"] = {"ms": r_ms, "tops": ops / r_ms / 1e9, "frac_int8_peak": ops / r_ms / 1e9 / PEAK_INT8}
    x_bytes = 4.0 * m * (h + i)
    out["per_token_quantizer_both_inputs"] = {"ms": q_ms, "gbps": (x_bytes + x_bytes / 4) / q_ms / 1e6}
    return out


def extra_host_path(layers, steps):
    """The W8A8 pair through the host-buffer entry (`rk_matmul`: f32 activations
    from and f32 outputs to ordinary pageable host arrays, quantized per 32-group
    on the GPU, as an unchanged Flex caller's `matmul` reaches it, ext.rs:1505-1554),
    PCIe included: the rate a caller that keeps its tensors in host memory sees."""
    xs = [np.ascontiguousarray(L["dx"].download((L["m"], L["k"]), np.float32)) for L in layers]
    ys = [np.empty((L["m"], L["n"]), np.float32) for L in layers]
    lib = rk.lib()

    def step():
        for L, x, y in zip(layers, xs, ys):
            call(lib.rk_matmul(int(L["wid"]), x.ctypes.data, L["m"], L["k"], y.ctypes.data), "rk_matmul")

    for _ in range(3):
        step()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    m, h, i = synth.W8A8["m"], synth.W8A8["hidden"], synth.W8A8["inter"]
    ops = 2 * 2.0 * m * h * i
    moved = sum(x.nbytes + y.nbytes for x, y in zip(xs, ys))
    return {"ms": ms, "tops": ops / ms / 1e9, "pcie_gbps": moved / ms / 1e6, "bytes_per_step": moved,
            "what": "rk_matmul on the up and down Q8_0 weights, host f32 in and out (group-32 activations)"}


def extra_glue(iters):
    """The HBM-bound ops around the GEMMs at the Qwen3-0.6B layer shape (S=3633, hidden 1024,
    MLP 3072, 16 q / 8 kv heads of 128): bytes are one read of each input and one write of
    each output."""
    c, g = synth.W8A8, synth.GQA_CAUSAL
    m, hid, inter = c["m"], c["hidden"], c["inter"]
    hq, hk, d = g["n_head"], g["n_kv"], g["d"]
    lib = rk.lib()
    r = np.random.default_rng(7)
    out = {}

    def rec(name, fn, nbytes):
        ms = time_launches(fn, iters)
        out[name] = {"ms": ms, "gbps": nbytes / ms / 1e6, "frac_hbm": nbytes / ms / 1e6 / PEAK_HBM}

    x16 = dev(r.standard_normal((m, hid)).astype(np.float16).view(np.uint16))
    w16 = dev((1 + 0.1 * r.standard_normal(hid)).astype(np.float16).view(np.uint16))
    y16 = rk.DeviceBuffer(m * hid * 2)
    rec("rms_norm_f16_3633x1024", lambda: call(lib.rk_rms_norm_dev(
        x16.ptr, w16.ptr, rk.DTYPE_F16, y16.ptr, m, hid, 1e-6, rk.DTYPE_F16, None), "rms"), 2 * m * hid * 2)
    width = (hq + 2 * hk) * d
    qkv = dev(r.standard_normal((m, width)).astype(np.float16).view(np.uint16))
    wq = dev((1 + 0.1 * r.standard_normal(d)).astype(np.float16).view(np.uint16))
    wk = dev((1 + 0.1 * r.standard_normal(d)).astype(np.float16).view(np.uint16))
    ang = np.arange(m)[:, None] * (10000.0 ** (-np.arange(d // 2) / (d // 2)))[None, :]
    cs = dev(np.cos(ang).astype(np.float16).view(np.uint16))
    sn = dev(np.sin(ang).astype(np.float16).view(np.uint16))
    rec("qk_norm_rope_f16_3633x4096", lambda: call(lib.rk_qk_norm_rope_dev(
        qkv.ptr, m, width, hq, hk, d, wq.ptr, wk.ptr, 1e-6, cs.ptr, sn.ptr, rk.DTYPE_F16, rk.DTYPE_F16, None),
        "qknr"), 2 * m * (hq + hk) * d * 2)
    o16 = rk.DeviceBuffer(m * hq * d * 2)
    ms = time_launches(lambda: call(lib.rk_attention_qkv_dev(
        qkv.ptr, m, width, hq, hk, d, wq.ptr, wk.ptr, 1e-6, cs.ptr, sn.ptr, rk.DTYPE_F16, d ** -0.5, 0.0, 1, -1,
        0, 0, o16.ptr, hq * d, None), "attention block"), iters)
    fl = attn_flops(m, m, hq, d, True)
    out["attention_block_qkv_3633"] = {"ms": ms, "tflops": fl / ms / 1e9, "frac_fp16_peak": fl / ms / 1e9 / PEAK_FP16}
    q8, qs8 = rk.DeviceBuffer(m * hid), rk.DeviceBuffer(m * 4)
    rec("rms_norm_quantize_f16_3633x1024", lambda: call(lib.rk_rms_norm_quantize_dev(
        x16.ptr, w16.ptr, rk.DTYPE_F16, m, hid, 1e-6, rk.DTYPE_F16, q8.ptr, qs8.ptr, None), "rmsq"),
        m * hid * 2 + m * hid + m * 4)
    n = m * inter
    a32, b32 = dev(r.standard_normal(n).astype(np.float32)), dev(r.standard_normal(n).astype(np.float32))
    o32 = rk.DeviceBuffer(n * 4)
    rec("silu_mul_f32_3633x3072", lambda: call(lib.rk_silu_mul_dev(
        a32.ptr, b32.ptr, o32.ptr, n, rk.DTYPE_F32, None), "silu"), 3 * n * 4)
    # per-token int8 activations of normal data, as in the headline workload
    xf = dev(synth.normal_f32(13, (m, hid)))
    xq, xs = rk.DeviceBuffer(m * hid), rk.DeviceBuffer(m * 4)
    call(lib.rk_quantize_rows_dev(xf.ptr, m, hid, hid, xq.ptr, xs.ptr, None), "quantize")
    gate = synth.normal_f32(11, (inter, hid), 0.02)
    up = synth.normal_f32(12, (inter, hid), 0.02)
    wid = rk.pack_q8_0_glu_f32(gate, up)
    ms = time_launches(lambda: call(lib.rk_matmul_w8a8_glu_dev(
        int(wid), xq.ptr, xs.ptr, m, hid, 1, o32.ptr, 0, None), "glu"), iters)
    ops = 2.0 * m * hid * 2 * inter
    out["w8a8_gate_up_silu_3633x1024x2x3072"] = {"ms": ms, "tops": ops / ms / 1e9,
                                                 "frac_int8_peak": ops / ms / 1e9 / PEAK_INT8}
    # fp16 gate|up GEMM with silu·up in its epilogue (f32 out), against the
    # unfused pair: the gate and up fp16 GEMMs, then silu_mul on their f32-widened outputs
    x16 = dev(synth.normal_f16(14, (m, hid)).view(np.uint16))
    wglu = rk.pack_f16_glu(gate, up)
    ms = time_launches(lambda: call(lib.rk_matmul_f16_glu_dev(int(wglu), x16.ptr, m, hid, 1, o32.ptr, 0, None),
                                    "f16 glu"), iters)
    out["f16_gate_up_silu_3633x1024x2x3072"] = {"ms": ms, "tflops": ops / ms / 1e9,
                                                "frac_fp16_peak": ops / ms / 1e9 / PEAK_FP16}
    wg, wu = rk.pack(gate), rk.pack(up)
    cg, cu = rk.DeviceBuffer(m * inter * 2), rk.DeviceBuffer(m * inter * 2)
    fg, fu = rk.DeviceBuffer(m * inter * 4), rk.DeviceBuffer(m * inter * 4)

    def unfused():
        call(lib.rk_matmul_f16_dev(int(wg), x16.ptr, m, hid, cg.ptr, None), "f16")
        call(lib.rk_matmul_f16_dev(int(wu), x16.ptr, m, hid, cu.ptr, None), "f16")
        call(lib.rk_cast_dev(cg.ptr, rk.DTYPE_F16, fg.ptr, rk.DTYPE_F32, m * inter, None), "widen")
        call(lib.rk_cast_dev(cu.ptr, rk.DTYPE_F16, fu.ptr, rk.DTYPE_F32, m * inter, None), "widen")
        call(lib.rk_silu_mul_dev(fg.ptr, fu.ptr, o32.ptr, m * inter, rk.DTYPE_F32, None), "silu")
    ms_u = time_launches(unfused, iters)
    out["f16_gate_up_silu_unfused_pair"] = {"ms": ms_u, "tflops": ops / ms_u / 1e9,
                                            "what": "two fp16 GEMMs, two f16->f32 widenings, silu_mul f32"}
    return out


# --------------------------------------------------------- CPU baseline ----
# The oracle's C restatement of each workload (the Burn flex CPU path cannot be
# built here), timed on the host cores in the same run: one warm-up call, then
# timed calls of a bounded sample until the time budget is spent; the median
# rate is the value, the best is reported beside it (the method of the
# reference's `gemm` command, src/commands/gemm.rs:76-104). Every workload is
# timed on all the cores this process may use and on one core.
def _host_threads():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def _time_cpu(fn, budget_s, min_reps=3, max_reps=40):
    fn()
    rates, spent = [], 0.0
    while (spent < budget_s or len(rates) < min_reps) and len(rates) < max_reps:
        t = time.perf_counter()
        work = fn()
        dt = time.perf_counter() - t
        rates.append(work / dt)
        spent += dt
    rates.sort()
    return rates[-1], rates[len(rates) // 2], spent, len(rates)


def _cpu_row(fn, unit, scale, sample_all, sample_one, budget_s):
    """fn(threads, one_core) runs one sample and returns its algorithmic work."""
    threads = _host_threads()
    b_all, m_all, t_all, n_all = _time_cpu(lambda: fn(threads, False), budget_s)
    b_one, m_one, t_one, n_one = _time_cpu(lambda: fn(1, True), budget_s)
    return {"value": m_all / scale, "best": b_all / scale, "unit": unit, "cores": threads, "kind": "port",
            "sample": f"{sample_all}; {n_all} timed runs, {t_all:.1f} s",
            "single_core": {"value": m_one / scale, "best": b_one / scale, "unit": unit, "cores": 1,
                            "sample": f"{sample_one}; {n_one} timed runs, {t_one:.1f} s"},
            "cpu": _cpu_model()}


def _spread_rows(n, chunks, width):
    """`chunks` runs of `width` rows spread evenly over [0, n)."""
    starts = np.linspace(0, n - width, chunks).round().astype(int)
    return [(int(a), int(a) + width) for a in starts]


def cpu_w8a8(oracle, budget_s):
    """Config 2: per-token quantize + the emu_matmul_gw formula (src/clef/int8.rs:101-158)."""
    c = synth.W8A8
    s1, s2, s3 = synth.SEEDS["w8a8"]
    data = []
    for (k, n, sx, sw) in ((c["hidden"], c["inter"], s1, s2), (c["inter"], c["hidden"], s1 + 1000, s3)):
        x = synth.normal_f32(sx, (c["m"], k))
        w = synth.normal_f32(sw, (n, k), 0.02)
        wq, wd = oracle.q8_0_quantize(w)
        data.append((x, wq, wd.view(np.float16).astype(np.float32), k))

    def fn(threads, one):
        rows = 192 if one else c["m"]
        ops = 0.0
        for x, wq, ws, k in data:
            aq, a_s = oracle.quantize_rows(x[:rows], k, threads)
            oracle.emu_matmul_gw(aq, a_s, k, wq, ws, 32, threads)
            ops += 2.0 * rows * k * wq.shape[0]
        return ops
    return _cpu_row(fn, "TOP/s", 1e12,
                    f"all {c['m']} rows of the up- and down-projection (per-token quantize + emu_matmul_gw), "
                    "OpenMP over rows", "192 rows of each projection", budget_s)


def cpu_gemm_f16(oracle, budget_s):
    """Config 1: fp16 inputs, f32 accumulation (src/commands/gemm.rs:79-83)."""
    c = synth.GEMM_F16
    s1, s2 = synth.SEEDS["gemm_f16"]
    a = synth.normal_f16(s1, (c["m"], c["k"]))
    b = synth.normal_f16(s2, (c["n"], c["k"]), 0.02)

    def fn(threads, one):
        rows = 48 if one else c["m"]
        oracle.gemm_f16(a[:rows], b, threads)
        return 2.0 * rows * c["n"] * c["k"]
    return _cpu_row(fn, "TFLOP/s", 1e12, f"the whole {c['m']}x{c['k']}x{c['n']} product",
                    f"48 rows of A", budget_s)


def _cpu_attention(oracle, s, h, kv, d, causal, seeds, budget_s, rows_all, rows_one):
    q = synth.normal_f16(seeds[0], (s, h * d))
    k = synth.normal_f16(seeds[1], (s, kv * d))
    v = synth.normal_f16(seeds[2], (s, kv * d))
    mode = 1 if causal else 0

    def fn(threads, one):
        chunks = _spread_rows(s, 8, (rows_one if one else rows_all) // 8)
        fl = 0.0
        for a, b in chunks:
            oracle.attention_flex(q[a:b], k, v, h, kv, d, d ** -0.5, 0.0, mode, -1, a, 0, threads)
            keys = (np.arange(a, b) + 1).sum() if causal else (b - a) * s
            fl += 4.0 * d * h * keys
        return fl
    what = (f"{{}} query rows in 8 runs spread over S={s} (TILE_KV=64 online-softmax flex restatement; "
            f"FLOPs of the visible keys only)")
    return _cpu_row(fn, "TFLOP/s", 1e12, what.format(rows_all), what.format(rows_one), budget_s)


def cpu_vision(oracle, budget_s):
    """Config 4: the four fp16 GEMMs on a row sample, and the attention."""
    c = synth.VISION
    s, hid, h, d, mlp = c["s"], c["hidden"], c["n_head"], c["d"], c["mlp"]
    seeds = synth.SEEDS["vision"]
    x = synth.normal_f16(seeds[0], (s, max(hid, mlp)))
    ws = [(synth.normal_f16(seeds[1 + i], (n, k), 0.02), k)
          for i, (n, k) in enumerate(((3 * hid, hid), (hid, hid), (mlp, hid), (hid, mlp)))]

    def fn(threads, one):
        rows = 16 if one else 256
        fl = 0.0
        for w, k in ws:
            oracle.gemm_f16(np.ascontiguousarray(x[:rows, :k]), w, threads)
            fl += 2.0 * rows * w.shape[0] * k
        return fl
    gemms = _cpu_row(fn, "TFLOP/s", 1e12, "256 of the 2394 rows through qkv, out, fc1 and fc2",
                     "16 rows through the four GEMMs", budget_s)
    att = _cpu_attention(oracle, s, h, h, d, False, seeds[6:9], budget_s, 128, 16)
    return {"gemms": gemms, "attention": att}


def cpu_moe(oracle, state, budget_s):
    """Config 5: the expert FFN of sampled tokens (orc_moe_experts: the reference's
    EmuWorker arithmetic, group-32 activations), and the 32/4-head attention."""
    c = synth.MOE
    S, H, E, K, I = c["s"], c["hidden"], c["experts"], c["top_k"], c["inter"]
    import concurrent.futures as cf
    threads = _host_threads()

    def q8(w):  # host Q8_0 of [E, rows, cols] in row chunks on a thread pool
        w2 = w.reshape(-1, w.shape[-1])
        q = np.empty(w2.shape, np.int8)
        dd = np.empty((w2.shape[0], w2.shape[1] // 32), np.float32)
        bounds = [(r, min(r + 4096, w2.shape[0])) for r in range(0, w2.shape[0], 4096)]

        def job(b):
            qq, d16 = oracle.q8_0_quantize(w2[b[0]:b[1]])
            q[b[0]:b[1]] = qq
            dd[b[0]:b[1]] = d16.view(np.float16).astype(np.float32)
        with cf.ThreadPoolExecutor(max_workers=threads) as ex:
            list(ex.map(job, bounds))
        return q.reshape(w.shape), dd.reshape(*w.shape[:-1], -1)
    (gq, gs), (uq, us), (dq, ds) = q8(state["gate"]), q8(state["up"]), q8(state["down"])
    x, ids, wts = state["x"], state["ids"], state["wts"]
    per_tok = 2.0 * K * (2 * I * H + H * I)

    def fn(threads_, one):
        toks = np.linspace(0, S - 1, 8 if one else 256).round().astype(np.int64)
        oracle.moe_experts(x[toks], ids[toks], wts[toks], gq, gs, uq, us, dq, ds, threads_)
        return per_tok * len(toks)
    experts = _cpu_row(fn, "TOP/s", 1e12, f"256 of the {S} tokens spread over the sequence, all {K} routed experts "
                       "each", "8 tokens", budget_s)
    att = _cpu_attention(oracle, S, c["attn_heads"], c["attn_kv"], c["attn_d"], True, synth.SEEDS["moe"][6:9],
                         budget_s, 128, 16)
    return {"experts": experts, "attention": att}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # ~65 ms of warm-up steps: the card's clocks take tens of ms of sustained work to settle
    # (100 steps, ~7 ms, leave the pair at 67 us per step against 60 us once settled)
    ap.add_argument("--warmup", type=int, default=1000)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=1.0,
                    help="timed CPU seconds per baseline row (all cores, then one core)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only the launches the rocprofv3 --pmc byte counts are taken from")
    ap.add_argument("--probe-all", action="store_true",
                    help="a few launches of every workload (for rocprofv3 --pmc counter runs)")
    ap.add_argument("--pmc-summary", nargs="+", metavar="CSV",
                    help="summarise rocprofv3 --pmc counter CSVs into profiles/traffic.json (no GPU)")
    a = ap.parse_args()
    if a.pmc_summary:
        pmc_summary(a.pmc_summary)
        return
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported on this single-GPU build "
              "(the multi-GPU sharding is a design note only)", file=sys.stderr)
        sys.exit(2)

    rk.init(0)
    name, cus, clk = rk.device_info()
    log(f"device {name}, {cus} CUs, {clk / 1e3:.0f} MHz")
    if a.probe_all:
        probe_all(5)
        return
    layers = setup_w8a8()
    if a.traffic_probe:
        traffic_probe(layers, TRAFFIC_LAUNCHES)
        return
    # The other device-resident workloads run first, then the headline: the
    # card's clocks take ~10 ms of sustained work to settle after the
    # host-side set-up, so a headline timed first after a few warm-up steps
    # (five are 0.3 ms of work) reads the power-state ramp rather than the
    # kernels. The headline's own W warm-up and K timed steps are unchanged;
    # they only come later. The extras that use the headline's buffers
    # re-quantize the same activations (per token, identical codes) and
    # overwrite only its output.
    extras = {}
    if not a.no_extras:
        for key, fn in (("w8a8_forms_3633", lambda: extra_w8a8_forms(layers, 50)),
                        ("gemm_f16_512x1024x3072", lambda: extra_gemm_f16(200)),
                        ("gqa_causal_3633", lambda: time_attention(
                            synth.GQA_CAUSAL["s"], synth.GQA_CAUSAL["n_head"], synth.GQA_CAUSAL["n_kv"],
                            synth.GQA_CAUSAL["d"], True, synth.SEEDS["gqa"], 50)),
                        ("vision_layer_2394", lambda: extra_vision(50)),
                        ("gemma_attention_d256_2587", lambda: extra_gemma_attention(50)),
                        ("moe_30b_a3b_1024", lambda: extra_moe(20)),
                        ("glue_qwen3_3633", lambda: extra_glue(50))):
            log(f"extra {key}")
            extras[key] = fn()

    log("W8A8 config ready; timing")
    ms, up_ms, wall = run_headline(layers, a.steps, a.warmup)
    m, h, i = synth.W8A8["m"], synth.W8A8["hidden"], synth.W8A8["inter"]
    ops_gemm = 2.0 * m * h * i
    value = 2 * ops_gemm / ms / 1e9
    achieved = ops_gemm / up_ms / 1e9
    log(f"step {ms:.4f} ms, up-proj {up_ms:.4f} ms, {value:.1f} TOP/s")
    if not a.no_extras:
        # after the headline: its PCIe copies leave the card mostly idle
        log("extra host_path_w8a8_pair_3633")
        extras["host_path_w8a8_pair_3633"] = extra_host_path(layers, 10)

    cpu = None
    if not a.no_cpu_baseline:
        sys.path.insert(0, ROOT)
        import oracle
        budget = a.cpu_seconds
        log("CPU baseline: W8A8 pair")
        cpu = cpu_w8a8(oracle, budget)
        if not a.no_extras:
            for key, fn in (("gemm_f16_512x1024x3072", lambda: cpu_gemm_f16(oracle, budget)),
                            ("gqa_causal_3633", lambda: _cpu_attention(
                                oracle, synth.GQA_CAUSAL["s"], synth.GQA_CAUSAL["n_head"], synth.GQA_CAUSAL["n_kv"],
                                synth.GQA_CAUSAL["d"], True, synth.SEEDS["gqa"], budget, 256, 32)),
                            ("vision_layer_2394", lambda: cpu_vision(oracle, budget)),
                            ("gemma_attention_d256_2587", lambda: _cpu_attention(
                                oracle, synth.GEMMA_TEXT["s"], synth.GEMMA_TEXT["n_head"], synth.GEMMA_TEXT["n_kv"],
                                synth.GEMMA_TEXT["d"], False, synth.SEEDS["gemma"], budget, 256, 32)),
                            ("moe_30b_a3b_1024", lambda: cpu_moe(oracle, _MOE_STATE, budget))):
                log(f"CPU baseline: {key}")
                extras[key]["cpu_baseline"] = fn()

    out = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: splitmix64 + Box-Muller normals, seeds " + str(synth.SEEDS["w8a8"]),
        "config": {"workload": "Q8_0/W8A8 MLP GEMMs, M=3633 tokens: up K=1024->N=3072 + down K=3072->N=1024, "
                               "per-token int8 activations, Q8_0 (32-value block) weights, f32 out",
                   "timed_region": "the two GEMM launches per step on int8 activations already quantized; the "
                                   "per-token quantizer runs before it (its time: extras.w8a8_forms_3633)",
                   "ops_per_step": 2 * ops_gemm, "sha256_x_up": layers[0]["sha_x"][:16],
                   "sha256_w_up": layers[0]["sha_w"][:16], "wall_s": round(wall, 4)},
        "roofline": {"bound": "mfma", "kernel": "gemm_i8_q8_kernel (up-projection 3633x1024->3072, per-token, f32 out)",
                     "achieved": round(achieved, 2), "peak": PEAK_INT8, "unit": "TOP/s",
                     "frac": round(achieved / PEAK_INT8, 4),
                     "frac_of_fp16_peak": round(achieved / PEAK_FP16, 4),
                     "limiter": "valu: the exact per-32-block scale fold, a convert and an FMA per output "
                                "element and block",
                     "ceilings": {"mfma_int8": PEAK_INT8, "valu_fold": round(VALU_FOLD_CEILING, 1)},
                     "frac_of_valu_fold_ceiling": round(achieved / VALU_FOLD_CEILING, 4),
                     "avg_launch_ms": round(up_ms, 5), "algorithmic_ops_per_launch": ops_gemm,
                     "traffic": load_traffic("w8a8_up")},
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
