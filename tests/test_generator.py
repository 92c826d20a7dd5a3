"""The synthetic-model generator's normal deviates (isa-lm_amd/csrc/kr_normal.h,
shared by the host C generator and the HIP generator) against the textbook
Box-Muller transform evaluated with numpy's float64 log / sqrt / cos / sin on
the same splitmix64 draws. CPU only; the device generator's bytes are checked
against the host's in tests/test_gpu_model.py."""
import numpy as np

import krafla as K

M64 = (1 << 64) - 1


def _mix64(z):
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _stream_key(seed, stream):
    with np.errstate(over="ignore"):
        z = np.uint64((seed * 0x9E3779B97F4A7C15 + stream * 0xD1B54A32D192ED03 + 0x632BE59BD9B4E019) & M64)
        return int(_mix64(z))


def _draws(key, n):
    with np.errstate(over="ignore"):
        j = np.arange(n, dtype=np.uint64)
        return _mix64(np.uint64(key) + (j + np.uint64(1)) * np.uint64(0x9E3779B97F4A7C15))


def _box_muller(z):
    u1 = ((z >> np.uint64(32)).astype(np.float64) + 0.5) / 4294967296.0
    u2 = ((z & np.uint64(0xFFFFFFFF)).astype(np.float64) + 0.5) / 4294967296.0
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * np.pi * u2
    return np.stack([r * np.cos(t), r * np.sin(t)], axis=1).reshape(-1)


def test_normals_match_textbook_box_muller():
    n = 1 << 21
    got = np.empty(n, dtype=np.float32)
    K.host.kr_gen_normal(got.ctypes.data, n, 9)   # stream 2000 of seed 9
    want64 = _box_muller(_draws(_stream_key(9, 2000), n // 2))
    want = want64.astype(np.float32)
    # the double values agree to ~1e-15 relative, so the floats are equal but
    # where the double lies within that of a rounding boundary
    diff = got != want
    assert np.count_nonzero(diff) <= n // 100000
    assert np.all(np.abs(got.astype(np.float64) - want64) <= 1e-6 * np.abs(want64) + 1e-30)


def test_normals_extremes():
    # the uniforms' ends: u1 = 2^-33 (the largest radius) and u1 -> 1; every
    # quadrant of the angle
    n = 1 << 16
    got = np.empty(n, dtype=np.float32)
    K.host.kr_gen_normal(got.ctypes.data, n, 12345)
    assert np.all(np.isfinite(got))
    assert np.abs(got).max() < 6.8   # sqrt(-2 ln 2^-33) = 6.76
    assert abs(float(got.mean())) < 0.02 and abs(float(got.std()) - 1.0) < 0.02
