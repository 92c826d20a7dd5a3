"""krh_attention_noalloc, the decode attention that allocates nothing (its
score rows live in a static device array), against krh_attention with a
caller-allocated workspace: bit for bit, on two calls in a row (the second
smaller, over the array's stale contents), and the size limit. Needs a
gfx950 device."""
import ctypes as C

import numpy as np
import pytest

import krafla as K

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(7)
SCRATCH_FLOATS = 1 << 21   # KRH_ATTN_SCRATCH_FLOATS


@pytest.fixture(scope="module", autouse=True)
def device():
    K.init_device()
    yield
    K.hip.krh_sync()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def both(nh, nkv, hd, max_seq, pos, window):
    """ao of krh_attention_noalloc and of krh_attention on the same inputs"""
    kvd, qd = nkv * hd, nh * hd
    q = K.DevBuf.of(RNG.normal(0, 1, qd).astype(np.float32))
    kc = K.DevBuf.of(RNG.normal(0, 1, max_seq * kvd).astype(np.float32))
    vc = K.DevBuf.of(RNG.normal(0, 1, max_seq * kvd).astype(np.float32))
    posb = K.DevBuf.of(np.array([pos], np.int32))
    scale = C.c_float(float(np.float32(1.0) / np.sqrt(np.float32(hd))))
    ao_n, ao_w, att = K.DevBuf(4 * qd), K.DevBuf(4 * qd), K.DevBuf(4 * nh * max_seq)
    K.hip.krh_attention_noalloc(ao_n.ptr, q.ptr, kc.ptr, vc.ptr, nh, nkv, hd, max_seq, window, scale, posb.ptr)
    K.hip.krh_attention(ao_w.ptr, None, None, att.ptr, q.ptr, kc.ptr, vc.ptr, nh, nkv, hd, max_seq, window, scale,
                        posb.ptr)
    st = K.hip.krh_sync()
    assert st == 0, K.hip.krh_last_error().decode()
    out = ao_n.get(np.float32, qd), ao_w.get(np.float32, qd)
    for b in (q, kc, vc, posb, ao_n, ao_w, att):
        b.free()
    return out


def test_noalloc_matches_workspace_entry_twice():
    # the 8B shape at a long position, then a smaller call (fewer heads, a
    # shorter cache and a window) over what the first left in the array
    for nh, nkv, hd, max_seq, pos, window in [(32, 8, 128, 4096, 3000, 0), (14, 2, 64, 1024, 500, 100)]:
        got, want = both(nh, nkv, hd, max_seq, pos, window)
        assert np.array_equal(bits(got), bits(want)), (nh, max_seq, pos)


def test_noalloc_rejects_beyond_the_array():
    nh, hd = 32, 128
    max_seq = SCRATCH_FLOATS // nh + 4   # one score row too long
    q = K.DevBuf(4 * nh * hd)
    ao = K.DevBuf(4 * nh * hd)
    posb = K.DevBuf.of(np.array([0], np.int32))
    K.hip.krh_attention_noalloc(ao.ptr, q.ptr, q.ptr, q.ptr, nh, 8, hd, max_seq, 0, C.c_float(0.1), posb.ptr)
    assert K.hip.krh_status() == K.ML_E_SHAPE
    assert b"scratch" in K.hip.krh_last_error()
    K.hip.krh_clear_error()
    assert K.hip.krh_sync() == 0
    for b in (q, ao, posb):
        b.free()
