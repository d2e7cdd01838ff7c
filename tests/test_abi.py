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
