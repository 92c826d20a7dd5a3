"""Parity at the workloads' full sizes. Needs a gfx950 device.

1. The three large workloads end to end against golden fixtures written by
   the reference's scalar build (tests/golden/make_config_golden.py: the
   reference's own ml_run, ISA=scalar, on the same model bytes): the model
   is regenerated on the device and must hash to the fixture's sha256; the
   greedy run must print the reference's ids; the teacher-forced logits of
   every position must equal the reference's bit for bit (hashed per row).
     - Qwen2.5-0.5B shape: 512-token prompt, 256 greedy tokens; tied Q4
       classifier (151936 x 896), QKV bias.
     - Llama-3.2-1B shape: 4000-token prompt, 96 greedy tokens to position
       4095 of the 4096-row cache; llama3 RoPE.
     - Llama-3-8B shape: 2048-token prompt prefilled in one batched step,
       256 greedy tokens; 128256 x 4096 Q8 classifier.
2. The batched kernels at the prompt lengths those workloads prefill (the
   pipelined main loop of the batched attention mix needs 256 or more
   attended positions), on the F32, F16 and Q8 caches; the MFMA matmul at
   2047 and 4000 tokens; the classifier matvec at both full vocabularies.
   Sampled tokens are checked against the oracle's per-position attention /
   matvec (a batched token's result is the decode result at its position)."""
import ctypes as C
import hashlib
import os
import shutil
import sys
import tempfile
import time

import numpy as np
import pytest

import krafla as K
import oracle_lib as O
from oracle_lib import oracle

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(2047)
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def say(msg):
    print("[fullsize] " + msg, file=sys.stderr, flush=True)


@pytest.fixture(scope="module", autouse=True)
def device():
    K.init_device()
    yield
    K.hip.krh_sync()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def ok():
    st = K.hip.krh_sync()
    assert st == 0, K.hip.krh_last_error().decode()


class Dev:
    def __init__(self):
        self.bufs = []

    def put(self, a):
        b = K.DevBuf.of(a)
        self.bufs.append(b)
        return b

    def zeros(self, nbytes):
        b = K.DevBuf(nbytes)
        self.bufs.append(b)
        return b

    def free(self):
        for b in self.bufs:
            b.free()


@pytest.fixture
def dev():
    d = Dev()
    yield d
    d.free()


# ---- 1. the workloads end to end ----

def scratch(nbytes):
    for d in ("/dev/shm", tempfile.gettempdir()):
        try:
            if shutil.disk_usage(d).free > nbytes + (2 << 30):
                return tempfile.mkdtemp(prefix="krfull_", dir=d)
        except OSError:
            pass
    return tempfile.mkdtemp(prefix="krfull_")


def file_sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            b = f.read(1 << 24)
            if not b:
                break
            h.update(b)
    return h.hexdigest()


def row_hashes(logits):
    out = np.empty(logits.shape[0], dtype=np.uint64)
    for i in range(logits.shape[0]):
        out[i] = np.frombuffer(hashlib.sha256(logits[i].tobytes()).digest()[:8], dtype="<u8")[0]
    return out


@pytest.mark.parametrize("name", ["qwen05b_mixed", "llama1b_mixed", "llama8b_q8"])
def test_workload_matches_reference(name):
    fx = os.path.join(GOLDEN, name + ".npz")
    if not os.path.exists(fx):
        pytest.skip("no golden fixture %s (tests/golden/make_config_golden.py writes it)" % fx)
    g = np.load(fx)
    tmp = scratch(int(g["mlb_bytes"]))
    try:
        path = os.path.join(tmp, name + ".mlb")
        t0 = time.time()
        K.gen_mlb(path, **dict(K.CONFIGS[name], device=1))
        say("%s: generated on the device in %.1f s" % (name, time.time() - t0))
        assert os.path.getsize(path) == int(g["mlb_bytes"])
        assert file_sha256(path) == str(g["mlb_sha256"]), "the device generator wrote other bytes"
        m = K.Model(path)
        s = K.State(m)
        try:
            ids, pre_s, dec_s = s.generate(g["prompt"], int(g["steps"]))
            say("%s: generated %d ids (prefill %.3f s, decode %.3f s)" % (name, len(ids), pre_s, dec_s))
            want = g["ids"]
            first = int(np.argmax(ids != want)) if not np.array_equal(ids, want) else -1
            assert np.array_equal(ids, want), "greedy ids differ from the reference's from index %d" % first
            forced = g["forced"]
            V = m.cfg.vocab
            logits = np.empty((forced.size, V), np.float32)
            s.prefill(forced, 0, logits=logits)
            h = row_hashes(logits)
            bad = np.nonzero(h != g["row_hash"])[0]
            if bad.size:
                am = np.argmax(logits, axis=1)
                say("%s: %d rows differ, first %d; argmax differs at %d rows; row max diff %g" % (
                    name, bad.size, bad[0], int(np.count_nonzero(am != g["argmax"])),
                    float(np.abs(logits.max(axis=1) - g["rowmax"]).max())))
                for p, ids_p, vals_p in zip(g["probe_pos"], g["probe_ids"], g["probe_vals"]):
                    rel = np.abs(logits[p][ids_p] - vals_p).max() / np.abs(vals_p).max()
                    say("%s: position %d: top-64 relative max-abs difference %g" % (name, p, rel))
            assert bad.size == 0, "%d of %d logits rows differ from the reference's" % (bad.size, forced.size)
            assert np.array_equal(np.argmax(logits, axis=1), g["argmax"])
        finally:
            s.close()
            m.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


@pytest.mark.parametrize("name", ["qwen05b_mixed", "llama1b_mixed", "llama8b_q8"])
def test_route_workload_matches_reference(name):
    """the reference's own ml_run over this backend's op table
    (oracle/_ref/hip/ml_run: model/transformer.c and app/ml_run.c unchanged,
    built with 2048-token prefill steps, the per-token op queue batching and
    fusing their calls) on the full-size model: the greedy ids the scalar
    build printed, and for the 0.5B shape every teacher-forced position's
    --dump-logits row against the fixture's hashes"""
    exe = os.path.join(O.REF_DIR, "hip", "ml_run")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref/hip not built (needs the reference sources at build time)")
    fx = os.path.join(GOLDEN, name + ".npz")
    if not os.path.exists(fx):
        pytest.skip("no golden fixture %s" % fx)
    g = np.load(fx)
    tmp = scratch(int(g["mlb_bytes"]) * 3)
    try:
        path = os.path.join(tmp, name + ".mlb")
        K.gen_mlb(path, **dict(K.CONFIGS[name], device=1))
        assert file_sha256(path) == str(g["mlb_sha256"]), "the device generator wrote other bytes"
        t0 = time.time()
        ids, err = O.ref_ml_run(path, g["prompt"], int(g["steps"]), isa="hip")
        say("%s: route ml_run %.1f s: %s" % (name, time.time() - t0, err.strip().splitlines()[-1][:120]))
        assert "isa: hip" in err
        want = g["ids"]
        first = int(np.argmax(ids != want)) if ids.shape == want.shape and not np.array_equal(ids, want) else -1
        assert np.array_equal(ids, want), "route ids differ from the reference's from index %d" % first
        if name == "qwen05b_mixed":
            forced = g["forced"]
            dump = os.path.join(tmp, "route.logits")
            O.ref_ml_run(path, forced, forced.size, dump=dump, isa="hip")
            V = K.CONFIGS[name]["vocab"]
            logits = np.fromfile(dump, dtype=np.float32).reshape(forced.size, V)
            bad = np.nonzero(row_hashes(logits) != g["row_hash"])[0]
            assert bad.size == 0, "%d of %d route logits rows differ, first %d" % (bad.size, forced.size,
                                                                                   bad[0] if bad.size else -1)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


# ---- 2. the batched kernels at the prompt lengths ----

def sample_tokens(T):
    """the tile and chunk edges, and 64 tokens spread evenly over the step"""
    picks = {0, 1, 62, 63, 64, 127, 128, 254, 255, 256, 257, 511, 512, 1023, T // 3, T // 2, T - 65, T - 64,
             T - 2, T - 1}
    picks |= {i * T // 64 + i % 7 for i in range(64)}
    return sorted(t for t in picks if 0 <= t < T)


def f16_rule(x):
    """half rounding of finite floats: numpy's round-to-nearest-even cast,
    the rule kro_f32_to_f16 follows (pinned in tests/test_oracle.py)"""
    return np.ascontiguousarray(x, np.float32).astype(np.float16).view(np.uint16)


def rand_cache(kv_type, max_seq, kvd, nkv):
    if kv_type == K.ML_F32:
        return f32(RNG.normal(0, 1, max_seq * kvd)), f32(RNG.normal(0, 1, max_seq * kvd)), None, None
    if kv_type == K.ML_F16:
        return f16_rule(RNG.normal(0, 1, max_seq * kvd)), f16_rule(RNG.normal(0, 1, max_seq * kvd)), None, None
    k = RNG.integers(-127, 128, max_seq * kvd).astype(np.int8)
    v = RNG.integers(-127, 128, max_seq * kvd).astype(np.int8)
    kd = f32(RNG.uniform(0.001, 0.05, max_seq * nkv))
    vd = f32(RNG.uniform(0.001, 0.05, max_seq * nkv))
    return k, v, kd, vd


def views(dev, kv_type, k, v, kd, vd):
    if kv_type == K.ML_F32:
        return (K.MlKvLayer(dev.put(k).ptr, dev.put(v).ptr, None, None, None, None, 0, None, None),
                O.KvLayer(k.ctypes.data, v.ctypes.data, None, None, None, None, 0, None, None))
    if kv_type == K.ML_F16:
        return (K.MlKvLayer(None, None, None, None, None, None, 0, dev.put(k).ptr, dev.put(v).ptr),
                O.KvLayer(None, None, None, None, None, None, 0, k.ctypes.data, v.ctypes.data))
    return (K.MlKvLayer(None, None, dev.put(k).ptr, dev.put(v).ptr, dev.put(kd).ptr, dev.put(vd).ptr, 0, None, None),
            O.KvLayer(None, None, k.ctypes.data, v.ctypes.data, kd.ctypes.data, vd.ctypes.data, 0, None, None))


@pytest.mark.parametrize("kv_type", [K.ML_F32, K.ML_F16, K.ML_Q8_0])
@pytest.mark.parametrize("nh,nkv,hd,T,max_seq", [(32, 8, 128, 2047, 2048), (32, 8, 64, 4000, 4000),
                                                 (14, 2, 64, 1000, 1024), (6, 6, 48, 300, 300)])
def test_attention_batch_prompt_lengths(dev, kv_type, nh, nkv, hd, T, max_seq):
    """a whole prompt's attention in one batched launch from position 0 (the
    last case ends at row max_seq - 1), every token (every third and the
    sampled ones over the Q8 cache, whose oracle is slower) bit-equal to the
    oracle's attention at its position"""
    kvd, qd = nkv * hd, nh * hd
    Q = f32(RNG.normal(0, 1, (T, qd)))
    k, v, kd, vd = rand_cache(kv_type, max_seq, kvd, nkv)
    dview, hview = views(dev, kv_type, k, v, kd, vd)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    ao, att = dev.zeros(4 * T * qd), dev.zeros(4 * T * nh * max_seq)
    K.hip.krh_attention_kv(ao.ptr, att.ptr, dev.put(Q).ptr, C.byref(dview), nh, nkv, hd, max_seq, scale,
                           dev.put(np.array([0], np.int32)).ptr, T, T - 1)
    ok()
    got = ao.get(np.float32, T * qd).reshape(T, qd)
    cfg = K.MlConfig(n_heads=nh, n_kv_heads=nkv, head_dim=hd, kv_dim=kvd, q_dim=qd, max_seq=max_seq,
                     attn_scale=scale)
    scratch_ = np.zeros(max_seq, np.float32)
    toks = range(T) if kv_type != K.ML_Q8_0 else sorted(set(range(0, T, 3)) | set(sample_tokens(T)))
    for t in toks:
        out = np.zeros(qd, np.float32)
        qt = f32(Q[t])
        oracle.kro_attention(out.ctypes.data, qt.ctypes.data, C.byref(hview), scratch_.ctypes.data, C.byref(cfg), t)
        assert np.array_equal(bits(got[t]), bits(out)), t


def rand_mat(rows, cols, typ):
    if typ == K.ML_Q8_0:
        q = RNG.integers(-127, 128, rows * cols, dtype=np.int8)
    else:
        q = RNG.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    dh = np.abs(RNG.normal(0, 0.01, rows * cols // 32)).astype(np.float16)
    return q, dh


def oracle_matvec(q, dh, rows, cols, typ, xq, xd):
    d = dh.astype(np.float32)
    W = O.qtensor(q, d, rows, cols, typ)
    y = np.zeros(rows, dtype=np.float32)
    fn = oracle.kro_matvec_q8 if typ == K.ML_Q8_0 else oracle.kro_matvec_q4
    fn(y.ctypes.data, C.byref(W), C.byref(O.qact(xq, xd)), 0, rows)
    return y


@pytest.mark.parametrize("typ,rows,cols,T", [(K.ML_Q8_0, 4096, 4096, 2047), (K.ML_Q8_0, 14336, 4096, 2047),
                                             (K.ML_Q8_0, 4096, 14336, 2047), (K.ML_Q4_0, 8192, 2048, 2048),
                                             (K.ML_Q8_0, 2048, 8192, 2048), (K.ML_Q4_0, 4864, 896, 511),
                                             # 128-row tiles from 3/4 of a tile per CU on: 336 and 192 tiles
                                             (K.ML_Q8_0, 14336, 4096, 300), (K.ML_Q4_0, 4096, 4096, 700),
                                             # 64-row tiles: a 128-token step of w1 (224 tiles)
                                             (K.ML_Q8_0, 14336, 4096, 128), (K.ML_Q4_0, 14336, 4096, 128)])
def test_matmul_prompt_lengths(dev, typ, rows, cols, T):
    """the prefill matmul over a whole prompt step: sampled tokens' rows
    bit-equal to the matvec (tests/test_kernels.c:146-189's rule)"""
    q, dh = rand_mat(rows, cols, typ)
    X = f32(RNG.normal(0, 1, (T, cols)) * RNG.choice([1e-2, 1.0, 30.0], (T, 1)))
    ldx = (T + 127) // 128 * 128
    xq_all, xd_all = O.quantize(X.ravel())
    nb = cols // 32
    xq = np.zeros((ldx, cols), np.int8)
    xq[:T] = xq_all.reshape(T, cols)
    xd = xd_all.reshape(T, nb)
    xdT = np.zeros((nb, ldx), np.float32)
    xdT[:, :T] = xd.T
    W = K.KrhMat(dev.put(q).ptr, dev.put(dh).ptr, rows, cols, typ, 1)
    y0 = f32(RNG.normal(0, 1, (T, rows)))
    yb = dev.put(y0)
    K.hip.krh_matmul(yb.ptr, rows, C.byref(W), dev.put(xq).ptr, dev.put(xdT).ptr, ldx, T, 1)
    ok()
    got = yb.get(np.float32, T * rows).reshape(T, rows)
    for t in sample_tokens(T):
        want = (y0[t] + oracle_matvec(q, dh, rows, cols, typ, xq[t], xd[t])).astype(np.float32)
        assert np.array_equal(bits(got[t]), bits(want)), t


@pytest.mark.parametrize("typ,rows,cols", [(K.ML_Q8_0, 128256, 4096), (K.ML_Q4_0, 151936, 896),
                                           (K.ML_Q4_0, 128256, 2048)])
def test_classifier_full_vocab(dev, typ, rows, cols):
    """the classifier launch (final rmsnorm + quantize + matvec,
    model/transformer.c:299-303) at the workloads' vocabularies, every row"""
    q, dh = rand_mat(rows, cols, typ)
    x = f32(RNG.normal(0, 3, cols))
    w = f32(RNG.normal(1, 0.1, cols))
    W = K.KrhMat(dev.put(q).ptr, dev.put(dh).ptr, rows, cols, typ, 1)
    yb = dev.zeros(4 * rows)
    K.hip.krh_rmsnorm_matvec(yb.ptr, C.byref(W), dev.put(x).ptr, dev.put(w).ptr, 1e-5, 0)
    ok()
    o = np.zeros(cols, np.float32)
    oracle.kro_rmsnorm(o.ctypes.data, x.ctypes.data, w.ctypes.data, cols, C.c_float(1e-5))
    xq, xd = O.quantize(o)
    assert np.array_equal(bits(yb.get(np.float32, rows)), bits(oracle_matvec(q, dh, rows, cols, typ, xq, xd)))
