"""The device sampler (krh_sample: the reference's ml_sample, model/sampler.c,
on device logits) against the oracle's sampler: over sequences of draws the
same ids, the same penalized logits and the same generator state, for every
option path and the inputs that steer them; then ml_run's sampled loop
(kr_generate with a sampler, graph replays) against the oracle's loop."""
import os

import numpy as np
import pytest

import krafla as K
import oracle_lib as O
from sampler_cases import KINDS, OPTS, gen_logits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    K.init_device()
    yield
    K.hip.krh_sync()


def ok():
    st = K.hip.krh_sync()
    assert st == 0, K.hip.krh_last_error().decode()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


class Bufs:
    def __init__(self):
        self.b = []

    def put(self, a):
        self.b.append(K.DevBuf.of(a))
        return self.b[-1]

    def free(self):
        for x in self.b:
            x.free()


def draws_match(n, opts, kind, draws, seed, vocab=None):
    """draws on the device and in the oracle from the same state; vocab > n
    leaves ids past n in the ring (the penalty skips them)"""
    vocab = vocab or n
    rng = np.random.default_rng(seed)
    bufs = Bufs()
    o, g = O.OracleSampler(vocab, opts), K.Sampler(vocab, opts)
    try:
        init = rng.integers(0, vocab + 3, 10).astype(np.int32)   # ids >= vocab are ignored
        for t in init:
            o.accept(t)
        g.accept(bufs.put(init).ptr, len(init))
        tb, pb, lb = bufs.put(np.zeros(1, np.int32)), bufs.put(np.zeros(1, np.int32)), bufs.put(
            np.full(draws + 2, -1, np.int32))
        want = []
        for k in range(draws):
            x = gen_logits(kind, n, rng)
            xo = x.copy()
            io = o.sample(xo)
            o.accept(io)
            want.append(io)
            xb = bufs.put(x)
            print("draw", n, kind, k, flush=True)
            g.sample(tb.ptr, xb.ptr, n, pb.ptr, lb.ptr)
            ok()
            assert tb.get(np.int32, 1)[0] == io, (kind, n, k)
            assert np.array_equal(bits(xb.get(np.float32, n)), bits(xo)), (kind, n, k)
            assert g.rng == o.rng, (kind, n, k)
        assert pb.get(np.int32, 1)[0] == draws
        assert np.array_equal(lb.get(np.int32, draws + 1)[1:], np.array(want, np.int32))
    finally:
        o.close()
        g.close()
        bufs.free()


@pytest.mark.parametrize("name", sorted(OPTS))
@pytest.mark.parametrize("n", [1, 2, 96, 1000, 32000])
def test_sample_matches_oracle(name, n):
    opts = O.sampler_opts(**OPTS[name])
    for k, kind in enumerate(KINDS):
        draws_match(n, opts, kind, 3, seed=7000 + 100 * n + k)


@pytest.mark.parametrize("name", ["mult", "topp", "topk", "topk_big", "greedy_penalty", "topp_tiny"])
def test_sample_matches_oracle_llama3_vocab(name):
    """128256 ids: the softmax's sum and the draws' sums over eleven groups,
    the sort over 126 workgroups"""
    opts = O.sampler_opts(**OPTS[name])
    for k, kind in enumerate(["normal", "ties", "tiny", "flat", "nan"]):
        draws_match(128256, opts, kind, 2, seed=99 + k)


def test_sample_n_below_vocab():
    """n < vocab: ring ids at or past n are not penalized (model/sampler.c:44)"""
    opts = O.sampler_opts(temperature=0.9, topp=0.8, repeat_penalty=1.7, repeat_last_n=32)
    draws_match(500, opts, "normal", 4, seed=3, vocab=520)


def test_sample_long_ring():
    """a ring longer than the workgroup (repeat_last_n 3000, many repeats)"""
    opts = O.sampler_opts(temperature=0.0, repeat_penalty=1.3, repeat_last_n=3000)
    rng = np.random.default_rng(8)
    n = 4000
    o, g = O.OracleSampler(n, opts), K.Sampler(n, opts)
    bufs = Bufs()
    try:
        ids = rng.integers(0, 700, 5000).astype(np.int32)
        for t in ids:
            o.accept(t)
        g.accept(bufs.put(ids).ptr, len(ids))
        tb = bufs.put(np.zeros(1, np.int32))
        for k in range(3):
            x = gen_logits("normal", n, rng)
            xo = x.copy()
            io = o.sample(xo)
            o.accept(io)
            xb = bufs.put(x)
            g.sample(tb.ptr, xb.ptr, n, None, None)
            ok()
            assert tb.get(np.int32, 1)[0] == io
            assert np.array_equal(bits(xb.get(np.float32, n)), bits(xo))
    finally:
        o.close()
        g.close()
        bufs.free()


def one_draw(opts, x, accepts=()):
    bufs = Bufs()
    g = K.Sampler(len(x), opts)
    try:
        if accepts:
            g.accept(bufs.put(np.array(accepts, np.int32)).ptr, len(accepts))
        tb, xb = bufs.put(np.zeros(1, np.int32)), bufs.put(np.ascontiguousarray(x, np.float32))
        g.sample(tb.ptr, xb.ptr, len(x), None, None)
        ok()
        return int(tb.get(np.int32, 1)[0]), xb.get(np.float32, len(x))
    finally:
        g.close()
        bufs.free()


def test_kat_reference_sampler_tests():
    """tests/test_sampler.c's answers on the device"""
    x = np.zeros(96, np.float32)
    x[40] = x[9] = 3.0
    assert one_draw(O.SamplerOpts(0.0, 0.9, 0, 1.0, 0, 1), x)[0] == 9
    x = np.zeros(96, np.float32)
    x[17] = 20.0
    assert one_draw(O.SamplerOpts(1.0, 0.5, 0, 1.0, 0, 3), x)[0] == 17
    x = np.zeros(96, np.float32)
    x[33] = 0.5
    assert one_draw(O.SamplerOpts(1.5, 0.9, 1, 1.0, 0, 9), x)[0] == 33
    x = np.zeros(96, np.float32)
    x[5], x[6], x[7] = 4.0, 3.0, -1.0
    t, y = one_draw(O.SamplerOpts(0.0, 0.0, 0, 2.0, 3, 1), x, accepts=(5, 5, 7))
    assert t == 6 and y[5] == 2.0 and y[7] == -2.0 and y[6] == 3.0


@pytest.mark.parametrize("name,extra", [
    ("topp", dict(temperature=0.8, topp=0.9, seed=11)),
    ("topk_penalty", dict(temperature=1.0, topk=20, topp=0.95, repeat_penalty=1.2, seed=3)),
    ("mult", dict(temperature=0.7, topp=1.0, seed=5)),
])
def test_generate_sampled_matches_oracle(name, extra, workdir):
    """kr_generate with a sampler (one graph replay per drawn id) against the
    oracle's ml_run loop, which the CPU tests pin to the reference's ml_run"""
    path = os.path.join(workdir, "smp_%s.mlb" % name)
    K.gen_mlb(path, **dict(K.CONFIGS["stories15m_q8"], std=0.1, seed=5))
    prompt = [1, 50, 300, 7]
    opts = O.sampler_opts(**extra)
    om = O.OracleModel(path)
    smp = O.OracleSampler(om.cfg.vocab, opts)
    want = om.generate_sampled(smp, prompt, 60)
    smp.close()
    om.close()
    m = K.Model(path)
    m.upload()
    st = K.State(m)
    st.set_sampler(opts)
    print("generate", name, flush=True)
    got, _, _ = st.generate(prompt, 60)
    assert np.array_equal(got, want)
    st.set_sampler(opts)   # a fresh sampler: the same draws again
    got2, _, _ = st.generate(prompt, 60)
    assert np.array_equal(got2, want)
    st.set_sampler(None)   # greedy again
    om = O.OracleModel(path)
    assert np.array_equal(st.generate(prompt, 30)[0], om.generate(prompt, 30))
    om.close()
    st.close()
    m.close()
