"""Seeded synthetic inputs for the five benchmark configurations.

A splitmix64 stream feeds a Box–Muller normal; values are produced in float64,
scaled to the requested sigma, rounded to float32 and then to fp16 with
round-to-nearest-even. The i-th 64-bit output of seed s is
mix(s + (i + 1)·0x9E3779B97F4A7C15), so the stream is vectorised with numpy's
wrapping uint64 arithmetic. Every configuration uses its own seeds; the
SHA-256 of each generated tensor identifies it in results.
"""
import concurrent.futures as cf
import hashlib
import os

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed, n, offset=0):
    """n outputs of the splitmix64 stream of `seed`, starting at output `offset`."""
    i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + i * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def uniform01(seed, n):
    """Doubles in [0, 1) from the top 53 bits."""
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def _normal_pairs(seed, p0, p1, sigma, out):
    """Box–Muller pairs [p0, p1) of the stream into out[2·p0 : 2·p1]."""
    bits = splitmix64(seed, 2 * (p1 - p0), offset=2 * p0)
    u = (bits >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * (p1 - p0), dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    out[2 * p0:2 * p1] = (z * sigma).astype(np.float32)


_CHUNK_PAIRS = 1 << 21


def normal(seed, n, sigma=1.0, threads=None):
    """n N(0, sigma²) samples as float32 (Box–Muller on consecutive pairs).

    The stream is counter based, so large requests are split into chunks that
    run on a thread pool (numpy releases the GIL); the values do not depend on
    the chunking."""
    pairs = (n + 1) // 2
    out = np.empty(2 * pairs, dtype=np.float32)
    bounds = [(p, min(p + _CHUNK_PAIRS, pairs)) for p in range(0, pairs, _CHUNK_PAIRS)]
    if len(bounds) <= 1:
        for p0, p1 in bounds:
            _normal_pairs(seed, p0, p1, sigma, out)
    else:
        workers = threads or min(16, os.cpu_count() or 1)
        with cf.ThreadPoolExecutor(max_workers=workers) as ex:
            list(ex.map(lambda b: _normal_pairs(seed, b[0], b[1], sigma, out), bounds))
    return out[:n]


def normal_f16(seed, shape, sigma=1.0):
    n = int(np.prod(shape))
    return normal(seed, n, sigma).astype(np.float16).reshape(shape)


def normal_f32(seed, shape, sigma=1.0):
    n = int(np.prod(shape))
    return normal(seed, n, sigma).reshape(shape)


def sha256(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ---------------------------------------------------------------- configs ----
# Shapes of the five configurations (sizes as named in the benchmark plan).
GEMM_F16 = dict(m=512, k=1024, n=3072)
W8A8 = dict(m=3633, hidden=1024, inter=3072)
GQA_CAUSAL = dict(s=3633, n_head=16, n_kv=8, d=128)
VISION = dict(s=2394, hidden=1152, n_head=16, d=72, mlp=4304)
MOE = dict(s=1024, hidden=2048, experts=128, top_k=8, inter=768, attn_heads=32, attn_kv=4, attn_d=128)
# EmbeddingGemma text attention: 3 query heads on one kv head of width 256, full
# layers and 512-key sliding layers, over a 2587-token document.
GEMMA_TEXT = dict(s=2587, n_head=3, n_kv=1, d=256, window=512)

SEEDS = {
    "gemm_f16": (101, 102),
    "w8a8": (201, 202, 203),
    "gqa": (301, 302, 303),
    "vision": (401, 402, 403, 404, 405, 406, 407, 408, 409),
    "moe": (501, 502, 503, 504, 505, 506, 507, 508, 509),
    "gemma": (601, 602, 603),
}
