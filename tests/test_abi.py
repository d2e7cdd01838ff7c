"""CPU tests of the C-ABI library: it loads, exports every declared entry point,
and its host-only logic (router, error reporting) behaves without a GPU."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "burn_rocket_amd.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rk_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_op_surface():
    names = _declared()
    for must in ("rk_init", "rk_pack", "rk_pack_seg", "rk_pack_i8", "rk_pack_q8_0", "rk_pack_qat",
                 "rk_matmul", "rk_matmul_f16_dev", "rk_matmul_w8a8_dev", "rk_matmul_i8_raw_dev",
                 "rk_attention", "rk_attention_dev", "rk_flash_attn_f16", "rk_moe_route",
                 "rk_moe_experts_dev", "rk_stats", "rk_mem_stats"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import burn_rocket
    lib = burn_rocket.load_library()
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    # the binding knows every entry point with a signature
    assert set(_declared()) == set(burn_rocket.SIGNATURES)


def test_calls_before_init_fail_loudly_without_a_device():
    import burn_rocket
    lib = burn_rocket.load_library()
    s = burn_rocket.Stats()
    rc = lib.rk_stats(ctypes.byref(s))
    if rc == 0:
        pytest.skip("engine already initialised in this process")
    assert rc == burn_rocket.RK_E_DEVICE
    assert b"rk_init" in lib.rk_last_error()


def test_fallback_classification():
    import burn_rocket
    lib = burn_rocket.load_library()
    # burn_rocket::Error::is_fallback (lib.rs:142-147): only the tiling status.
    assert lib.rk_is_fallback(-2) == 1
    assert lib.rk_is_fallback(-1) == 0 and lib.rk_is_fallback(-4) == 0


def test_router_matches_the_oracle(orc):
    import burn_rocket
    burn_rocket.load_library()
    r = np.random.default_rng(3)
    logits = r.standard_normal((257, 128)).astype(np.float32)
    logits[7, :] = 0.25  # ties resolve to the lower id
    for norm in (True, False):
        ids, wts = burn_rocket.moe_route(logits, 8, norm)
        oids, owts = orc.route(logits, 8, norm)
        assert (ids == oids).all()
        assert np.allclose(wts, owts, rtol=2e-6, atol=1e-8)
    assert list(ids[7]) == list(range(8))


def test_router_rejects_bad_top_k():
    import burn_rocket
    burn_rocket.load_library()
    with pytest.raises(burn_rocket.RocketError) as e:
        burn_rocket.moe_route(np.zeros((2, 4), np.float32), 5)
    assert e.value.rc == burn_rocket.RK_E_SHAPE


def _mask(n_q, n_kv, keep):
    i = np.arange(n_q)[:, None]
    j = np.arange(n_kv)[None, :]
    return np.ascontiguousarray(np.where(np.broadcast_to(keep(i, j), (n_q, n_kv)), np.float16(0), np.float16(-np.inf)).astype(np.float16))


def test_additive_mask_classification_without_a_device():
    # rk_flash_attn_f16_masked reads the mask on the host before it touches the
    # device: the reference builders' masks (masks.rs:11-114) pass to the
    # device stage (RK_E_DEVICE here, no engine), other masks are refused.
    import burn_rocket
    lib = burn_rocket.load_library()
    s = burn_rocket.Stats()
    if lib.rk_stats(ctypes.byref(s)) == 0:
        pytest.skip("engine already initialised in this process")
    z = np.zeros(4096, np.uint16)

    def rc(mask, n_q, n_kv):
        return lib.rk_flash_attn_f16_masked(n_q, n_kv, 64, 64, 1, 1, 0.125, 0.0, mask.view(np.uint16).ctypes.data,
                                            z.ctypes.data, z.ctypes.data, z.ctypes.data, z.ctypes.data)

    good = [(_mask(40, 40, lambda i, j: j <= i), 40, 40),
            (_mask(40, 40, lambda i, j: np.abs(i - j) <= 3), 40, 40),
            (_mask(40, 40, lambda i, j: (j <= i) & (j > i - 5)), 40, 40),
            (_mask(24, 64, lambda i, j: j <= i + 30), 24, 64),                       # causal block
            (_mask(24, 64, lambda i, j: np.abs((50 + i) - (20 + j)) <= 9), 24, 64),   # band block
            (_mask(24, 64, lambda i, j: (j <= i + 30) & (j > i + 30 - 12)), 24, 64),  # causal window block
            (_mask(16, 64, lambda i, j: j < 0), 16, 64),                              # every row hidden
            (_mask(16, 64, lambda i, j: j >= 0), 16, 64)]                             # nothing hidden
    for m, n_q, n_kv in good:
        assert rc(m, n_q, n_kv) == burn_rocket.RK_E_DEVICE, lib.rk_last_error()
    bad = [(np.full((40, 40), -2.0, np.float16), 40, 40),                  # a finite bias
           (_mask(40, 40, lambda i, j: (j % 3) != 1), 40, 40),              # several intervals per row
           (_mask(40, 40, lambda i, j: (i % 2 == 0) | (j < 0)), 40, 40),    # full and empty rows alternate
           (_mask(40, 40, lambda i, j: j <= i // 2), 40, 40)]               # a band that widens
    for m, n_q, n_kv in bad:
        assert rc(m, n_q, n_kv) == burn_rocket.RK_E_UNSUPPORTED
        assert b"mask" in lib.rk_last_error()
