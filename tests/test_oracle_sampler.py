"""The oracle's sampler (oracle/kro.c, kro_sample) pinned against the
reference's own ml_sample (model/sampler.c, built into oracle/_ref) and the
known answers of the reference's tests/test_sampler.c. CPU only."""
import os

import numpy as np
import pytest

import krafla as K
import oracle_lib as O
from oracle_lib import ref
from sampler_cases import INF, KINDS, OPTS, gen_logits

needs_ref = pytest.mark.skipif(ref is None, reason="oracle/_ref not built (needs the reference sources)")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def run_pair(n, opts, kind, draws, seed):
    rng = np.random.default_rng(seed)
    o, r = O.OracleSampler(n, opts), O.ReferenceSampler(n, opts)
    for t in rng.integers(0, n + 3, 10):   # ids at or past vocab are ignored
        o.accept(t)
        r.accept(t)
    for _ in range(draws):
        x = gen_logits(kind, n, rng)
        xo, xr = x.copy(), x.copy()
        io, ir = o.sample(xo), r.sample(xr)
        assert io == ir, (kind, n)
        assert np.array_equal(bits(xo), bits(xr))   # the penalty's writes
        assert o.rng == r.rng
        assert 0 <= io < n
        o.accept(io)
        r.accept(ir)
    o.close()
    r.close()


@needs_ref
@pytest.mark.parametrize("name", sorted(OPTS))
@pytest.mark.parametrize("n", [1, 2, 96, 1000])
def test_sampler_matches_reference(name, n):
    opts = O.sampler_opts(**OPTS[name])
    for k, kind in enumerate(KINDS):
        run_pair(n, opts, kind, 6, seed=1000 * n + k)


@needs_ref
@pytest.mark.parametrize("name", ["mult", "topp", "topk", "topk_big"])
def test_sampler_matches_reference_large_vocab(name):
    opts = O.sampler_opts(**OPTS[name])
    for k, kind in enumerate(["normal", "ties", "tiny"]):
        run_pair(32000, opts, kind, 3, seed=77 + k)


# tests/test_sampler.c's known answers, on the oracle
def test_kat_topp_empty_nucleus():
    s = O.OracleSampler(96, O.SamplerOpts(1.0, 1e-6, 0, 1.0, 0, 7))
    for _ in range(50):
        assert 0 <= s.sample(np.zeros(96, np.float32)) < 96
    s.close()


def test_kat_topp_picks_from_nucleus():
    s = O.OracleSampler(96, O.SamplerOpts(1.0, 0.5, 0, 1.0, 0, 3))
    for _ in range(50):
        x = np.zeros(96, np.float32)
        x[17] = 20.0
        assert s.sample(x) == 17
    s.close()


def test_kat_greedy_ties_lowest():
    s = O.OracleSampler(96, O.SamplerOpts(0.0, 0.9, 0, 1.0, 0, 1))
    x = np.zeros(96, np.float32)
    x[40] = x[9] = 3.0
    assert s.sample(x) == 9
    s.close()


def test_kat_topk():
    s = O.OracleSampler(96, O.SamplerOpts(2.0, 0.0, 3, 1.0, 0, 5))
    seen = np.zeros(96, int)
    for _ in range(400):
        x = ((np.arange(96) % 7) * np.float32(0.1)).astype(np.float32)
        x[10], x[50], x[80] = 1.0, 0.95, 0.9
        seen[s.sample(x)] += 1
    assert seen[10] + seen[50] + seen[80] == 400 and min(seen[10], seen[50], seen[80]) > 0
    s.close()
    s = O.OracleSampler(96, O.SamplerOpts(1.5, 0.9, 1, 1.0, 0, 9))
    for _ in range(50):
        x = np.zeros(96, np.float32)
        x[33] = 0.5
        assert s.sample(x) == 33
    s.close()


def test_kat_repeat_penalty():
    s = O.OracleSampler(96, O.SamplerOpts(0.0, 0.0, 0, 2.0, 3, 1))
    x = np.zeros(96, np.float32)
    x[5], x[6], x[7] = 4.0, 3.0, -1.0
    assert s.sample(x) == 5
    for t in (5, 5, 7):
        s.accept(t)
    x = np.zeros(96, np.float32)
    x[5], x[6], x[7] = 4.0, 3.0, -1.0
    assert s.sample(x) == 6
    assert x[5] == 2.0 and x[7] == -2.0 and x[6] == 3.0
    for t in (1, 2, 3):
        s.accept(t)
    x = np.zeros(96, np.float32)
    x[5], x[6] = 4.0, 3.0
    assert s.sample(x) == 5
    s.close()


def test_multinomial_walk_closed_form():
    """with one token holding all the mass (the others -inf), every draw is it;
    with two equal halves, a draw below 0.5 is the first (the coin's 24-bit
    grid makes 0.5 itself the second)"""
    s = O.OracleSampler(8, O.sampler_opts(temperature=1.0, topp=1.0, seed=3))
    for _ in range(20):
        x = np.full(8, -INF, np.float32)
        x[5] = 1.0
        assert s.sample(x) == 5
    s.close()
    seen = set()
    s = O.OracleSampler(2, O.sampler_opts(temperature=1.0, topp=1.0, seed=9))
    for _ in range(200):
        seen.add(s.sample(np.zeros(2, np.float32)))
    assert seen == {0, 1}
    s.close()


@needs_ref
def test_generate_sampled_matches_ml_run(workdir):
    """ml_run -T 0.8 -p 0.9 (and --top-k 20, --repeat-penalty 1.2) on a
    generated model: the ids it prints equal the oracle's loop"""
    path = os.path.join(workdir, "smp_c1.mlb")
    K.gen_mlb(path, **dict(K.CONFIGS["stories15m_q8"], std=0.1, seed=5))
    prompt = [1, 50, 300, 7]
    for extra, opts in [
        (["-T", "0.8", "-p", "0.9", "-s", "11"], O.sampler_opts(temperature=0.8, topp=0.9, seed=11)),
        (["-T", "1.0", "--top-k", "20", "-p", "0.95", "--repeat-penalty", "1.2", "-s", "3"],
         O.sampler_opts(temperature=1.0, topk=20, topp=0.95, repeat_penalty=1.2, seed=3)),
    ]:
        ids_ref, _ = O.ref_ml_run(path, prompt, 40, extra=extra)
        om = O.OracleModel(path)
        smp = O.OracleSampler(om.cfg.vocab, opts)
        assert np.array_equal(om.generate_sampled(smp, prompt, 40), ids_ref)
        smp.close()
        om.close()
