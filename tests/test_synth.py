"""The seeded input generator: splitmix64 known answers and the normal law."""
import numpy as np

from burn_rocket import synth


def test_splitmix64_known_answers():
    # Published splitmix64 outputs for seed 0 (Vigna's reference generator).
    got = [int(x) for x in synth.splitmix64(0, 3)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    # offset continues the same stream
    assert int(synth.splitmix64(0, 1, offset=2)[0]) == got[2]


def test_normal_is_standard_and_deterministic():
    z = synth.normal(123, 1_000_001)
    assert z.dtype == np.float32 and z.size == 1_000_001
    assert abs(float(z.mean())) < 5e-3 and abs(float(z.std()) - 1) < 5e-3
    assert (synth.normal(123, 10) == z[:10]).all()
    w = synth.normal_f16(7, (64, 32), 0.02)
    assert w.dtype == np.float16 and abs(float(w.astype(np.float32).std()) - 0.02) < 2e-3
    assert synth.sha256(w) == synth.sha256(synth.normal_f16(7, (64, 32), 0.02))
