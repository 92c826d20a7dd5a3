"""The F16 and Q8 KV caches on the device: the cache rounding and
quantization (store_kv, model/transformer.c:191-205), attention over them
(ops/ops.c:124-180, k_scalar.c:124-155) against the oracle, bit for bit, and
the whole token loop against the reference's own ml_run --kv f16|q8. Needs a
gfx950 device."""
import ctypes as C
import os

import numpy as np
import pytest

import krafla as K
import oracle_lib as O
from oracle_lib import oracle
from test_gpu_kernels import Dev, bits, f32, ok
from test_gpu_model import SMALL

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(77)
KRH_MATH_F2H = 4   # include/krafla_hip.h: the F16 cache's rounding


@pytest.fixture(scope="module", autouse=True)
def device():
    K.init_device()
    yield
    K.hip.krh_sync()


@pytest.fixture
def dev():
    d = Dev()
    yield d
    d.free()


def f16_rule(x):
    """the oracle's half rounding (kro_f32_to_f16, pinned on the CPU against
    the IEEE conversion on every input): numpy's round-to-nearest-even cast,
    NaN to sign | 0x7e00"""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32)
    with np.errstate(over="ignore", invalid="ignore"):
        h = x.astype(np.float16).view(np.uint16)
    return np.where(np.isnan(x), ((u >> 16) & 0x8000).astype(np.uint16) | np.uint16(0x7E00), h)


def test_f16_rounding_matches_oracle(dev):
    """the device's half rounding on a million random bit patterns and every
    pattern next to the subnormal, normal, overflow and NaN boundaries"""
    edges = [0x33000000, 0x38800000, 0x477FE000, 0x477FF000, 0x7F800000]
    u = np.concatenate([RNG.integers(0, 1 << 32, 1 << 20, dtype=np.uint64)] +
                       [np.arange(e - 4096, e + 4096, dtype=np.uint64) for e in edges]).astype(np.uint32)
    u = np.concatenate([u, u ^ np.uint32(0x80000000)])
    x = u.view(np.float32)
    y = dev.zeros(4 * len(x))
    K.hip.krh_math_batch(KRH_MATH_F2H, y.ptr, dev.put(x).ptr, None, len(x))
    ok()
    got = (y.get(np.float32, len(x)).view(np.uint32) & 0xFFFF).astype(np.uint16)
    want = f16_rule(x)
    chunk = np.empty(1, np.uint16)
    for i in range(0, len(x), 997):   # spot-check the rule against the oracle itself
        oracle.kro_f32_to_f16_range(chunk.ctypes.data, int(u[i]), 1)
        assert chunk[0] == want[i]
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, "bits %#x: device %#x, want %#x" % (u[bad[0]], got[bad[0]], want[bad[0]])


@pytest.mark.parametrize("kv_type", [K.ML_F16, K.ML_Q8_0])
@pytest.mark.parametrize("nkv,hd,pos0,T", [(8, 128, 0, 1), (8, 128, 2175, 1), (2, 64, 37, 19), (1, 48, 5, 3)])
def test_store_kv(dev, kv_type, nkv, hd, pos0, T):
    max_seq = pos0 + T + 3
    kvd = nkv * hd
    k = f32(RNG.normal(0, 1, (T, kvd)) * RNG.choice([1e-6, 1.0, 300.0], (T, kvd)))
    v = f32(RNG.normal(0, 2, (T, kvd)))
    k[0, :hd] = 0.0    # an all-zero head: scale 0, quants 0
    es = 2 if kv_type == K.ML_F16 else 1
    kc, vc = dev.zeros(es * max_seq * kvd), dev.zeros(es * max_seq * kvd)
    kd, vd = dev.zeros(4 * max_seq * nkv), dev.zeros(4 * max_seq * nkv)
    K.hip.krh_store_kv(kv_type, kc.ptr, vc.ptr, kd.ptr if kv_type == K.ML_Q8_0 else None,
                       vd.ptr if kv_type == K.ML_Q8_0 else None, dev.put(k).ptr, dev.put(v).ptr, nkv, hd,
                       dev.put(np.array([pos0], np.int32)).ptr, T)
    ok()
    for src, cache, scales in ((k, kc, kd), (v, vc, vd)):
        if kv_type == K.ML_F16:
            got = cache.get(np.uint16, max_seq * kvd).reshape(max_seq, kvd)[pos0:pos0 + T]
            assert np.array_equal(got.ravel(), f16_rule(src.ravel()))
        else:
            got = cache.get(np.int8, max_seq * kvd).reshape(max_seq, kvd)[pos0:pos0 + T]
            gd = scales.get(np.float32, max_seq * nkv).reshape(max_seq, nkv)[pos0:pos0 + T]
            for t in range(T):
                for h in range(nkv):
                    q, d = np.zeros(hd, np.int8), np.zeros(1, np.float32)
                    row = f32(src[t, h * hd:(h + 1) * hd])
                    oracle.kro_quantize_row(q.ctypes.data, d.ctypes.data, row.ctypes.data, hd)
                    assert np.array_equal(got[t, h * hd:(h + 1) * hd], q) and bits(gd[t, h])[()] == bits(d)[0]


def rand_cache(kv_type, max_seq, kvd, nkv):
    """a random cache of the type: halves rounded from normal floats, or int8
    rows with positive row scales"""
    if kv_type == K.ML_F16:
        k = f16_rule(RNG.normal(0, 1, max_seq * kvd))
        v = f16_rule(RNG.normal(0, 1, max_seq * kvd))
        return k, v, None, None
    k = RNG.integers(-127, 128, max_seq * kvd).astype(np.int8)
    v = RNG.integers(-127, 128, max_seq * kvd).astype(np.int8)
    kd = f32(RNG.uniform(0.001, 0.05, max_seq * nkv))
    vd = f32(RNG.uniform(0.001, 0.05, max_seq * nkv))
    return k, v, kd, vd


def views(dev, kv_type, k, v, kd, vd, window):
    """the cache as an ml_kv_layer of device pointers and of host pointers"""
    if kv_type == K.ML_F16:
        return (K.MlKvLayer(None, None, None, None, None, None, window, dev.put(k).ptr, dev.put(v).ptr),
                O.KvLayer(None, None, None, None, None, None, window, k.ctypes.data, v.ctypes.data))
    return (K.MlKvLayer(None, None, dev.put(k).ptr, dev.put(v).ptr, dev.put(kd).ptr, dev.put(vd).ptr, window, None,
                        None),
            O.KvLayer(None, None, k.ctypes.data, v.ctypes.data, kd.ctypes.data, vd.ctypes.data, window, None, None))


@pytest.mark.parametrize("kv_type", [K.ML_F16, K.ML_Q8_0])
@pytest.mark.parametrize("nh,nkv,hd,pos,window", [(6, 6, 48, 0, 0), (14, 2, 64, 511, 0), (32, 8, 128, 2175, 0),
                                                  (32, 8, 128, 2303, 0), (8, 2, 64, 100, 7), (16, 1, 64, 63, 0),
                                                  (12, 4, 96, 130, 0), (4, 2, 32, 9000, 0), (8, 4, 256, 300, 0),
                                                  (4, 1, 256, 200, 64), (32, 8, 128, 4095, 0), (8, 8, 64, 1000, 0)])
def test_attention_kv(dev, kv_type, nh, nkv, hd, pos, window):
    max_seq = max(256, pos + 1)
    kvd, qd = nkv * hd, nh * hd
    q = f32(RNG.normal(0, 1, qd))
    q[:hd] = 0.0   # a zero query head: Q8 scale 0
    k, v, kd, vd = rand_cache(kv_type, max_seq, kvd, nkv)
    dview, hview = views(dev, kv_type, k, v, kd, vd, window)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    ao, att = dev.zeros(4 * qd), dev.zeros(4 * nh * max_seq)
    K.hip.krh_attention_kv(ao.ptr, att.ptr, dev.put(q).ptr, C.byref(dview), nh, nkv, hd, max_seq, scale,
                           dev.put(np.array([pos], np.int32)).ptr, 1, max_seq - 1)
    ok()
    cfg = K.MlConfig(n_heads=nh, n_kv_heads=nkv, head_dim=hd, kv_dim=kvd, q_dim=qd, max_seq=max_seq,
                     attn_scale=scale)
    out = np.zeros(qd, np.float32)
    scratch = np.zeros(max_seq, np.float32)
    oracle.kro_attention(out.ctypes.data, q.ctypes.data, C.byref(hview), scratch.ctypes.data, C.byref(cfg), pos)
    assert np.array_equal(bits(ao.get(np.float32, qd)), bits(out))


@pytest.mark.parametrize("kv_type", [K.ML_F16, K.ML_Q8_0])
@pytest.mark.parametrize("nh,nkv,hd,pos0,T,window", [(6, 6, 48, 0, 40, 0), (32, 8, 128, 100, 70, 0),
                                                     (14, 2, 64, 3, 200, 0), (8, 2, 64, 10, 50, 7),
                                                     (8, 4, 256, 5, 40, 0), (4, 1, 256, 100, 30, 64),
                                                     (16, 8, 64, 7, 45, 0), (8, 8, 128, 200, 70, 0)])
@pytest.mark.parametrize("rb", [False, True])
def test_attention_kv_batch(dev, kv_type, nh, nkv, hd, pos0, T, window, rb):
    """batched attention over F16 and Q8 caches against the oracle's per-token
    attention; rb: the register-blocked kernels forced on (64- and 128-dim
    heads; at these sizes the launch would take the per-token-block kernels)"""
    if rb and hd not in (64, 128):
        pytest.skip("the register-blocked kernels take 64- and 128-dim heads")
    if rb:
        K.hip.krh_set_attn_rb_min(0)
    try:
        kv_batch_case(dev, kv_type, nh, nkv, hd, pos0, T, window)
    finally:
        K.hip.krh_set_attn_rb_min(512)


@pytest.mark.parametrize("nh,nkv,hd,pos0,T", [(32, 2, 256, 5, 40), (16, 2, 512, 0, 20)])
def test_attention_kv_batch_q8_wide_groups(dev, nh, nkv, hd, pos0, T):
    """the batched Q8 score kernel when a group's quantized queries leave room
    for 8 (group 16, head 256) or 4 (group 8, head 512) tokens a pass; the F16
    score tile of these heads does not fit in 64 KB of LDS"""
    kv_batch_case(dev, K.ML_Q8_0, nh, nkv, hd, pos0, T, 0)


def kv_batch_case(dev, kv_type, nh, nkv, hd, pos0, T, window):
    max_seq = 512
    kvd, qd = nkv * hd, nh * hd
    Q = f32(RNG.normal(0, 1, (T, qd)))
    k, v, kd, vd = rand_cache(kv_type, max_seq, kvd, nkv)
    dview, hview = views(dev, kv_type, k, v, kd, vd, window)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    ao, att = dev.zeros(4 * T * qd), dev.zeros(4 * T * nh * max_seq)
    K.hip.krh_attention_kv(ao.ptr, att.ptr, dev.put(Q).ptr, C.byref(dview), nh, nkv, hd, max_seq, scale,
                           dev.put(np.array([pos0], np.int32)).ptr, T, pos0 + T - 1)
    ok()
    got = ao.get(np.float32, T * qd).reshape(T, qd)
    cfg = K.MlConfig(n_heads=nh, n_kv_heads=nkv, head_dim=hd, kv_dim=kvd, q_dim=qd, max_seq=max_seq,
                     attn_scale=scale)
    scratch = np.zeros(max_seq, np.float32)
    for t in range(T):
        out = np.zeros(qd, np.float32)
        qt = f32(Q[t])
        oracle.kro_attention(out.ctypes.data, qt.ctypes.data, C.byref(hview), scratch.ctypes.data, C.byref(cfg),
                             pos0 + t)
        assert np.array_equal(bits(got[t]), bits(out)), t


KV = {"f16": K.ML_F16, "q8": K.ML_Q8_0}


@pytest.mark.parametrize("batch", [0, 1, 5])
@pytest.mark.parametrize("kv", sorted(KV))
@pytest.mark.parametrize("name", ["c1_q8", "llama3_rope_gqa_q4", "qwen_like_q4mix", "q8_f16_untied"])
def test_logits_match_reference_kv(name, kv, batch, workdir):
    """logits of every prompt position against ml_run --kv (app/ml_run.c:277-281),
    through batched prefill (batch 0: the default step), token by token (1)
    and chunks of 5"""
    path = os.path.join(workdir, name + ".mlb")
    if not os.path.exists(path):
        K.gen_mlb(path, **SMALL[name])
    m = K.Model(path)
    s = K.State(m, KV[kv])
    if batch:
        s.set_batch(batch)
    V = m.cfg.vocab
    toks = [int(t) for t in np.random.default_rng(6).integers(1, V, 12)]
    dump = path + "." + kv + ".logits"
    if not os.path.exists(dump):
        O.ref_ml_run(path, toks, len(toks), dump=dump, extra=("--kv", kv))
    want = np.fromfile(dump, dtype=np.float32).reshape(len(toks), V)
    got = np.empty((len(toks), V), dtype=np.float32)
    s.prefill(toks, 0, logits=got)
    assert np.array_equal(bits(got), bits(want))
    s.close()
    m.close()


@pytest.mark.parametrize("kv", sorted(KV))
@pytest.mark.parametrize("name", ["c1_q8", "llama3_rope_gqa_q4", "q8_f16_untied"])
def test_greedy_ids_match_reference_kv(name, kv, workdir):
    path = os.path.join(workdir, name + ".mlb")
    if not os.path.exists(path):
        K.gen_mlb(path, **SMALL[name])
    m = K.Model(path)
    s = K.State(m, KV[kv])
    toks = [int(t) for t in np.random.default_rng(6).integers(1, m.cfg.vocab, 5)]
    steps = min(m.cfg.max_seq, 60)
    ids_ref, _ = O.ref_ml_run(path, toks, steps, extra=("--kv", kv))
    ids, _, _ = s.generate(toks, steps)
    assert np.array_equal(ids, ids_ref)
    s.close()
    m.close()


@pytest.mark.parametrize("dim,nh,nkv,hd,typ,vtyp,bias", [(896, 14, 2, 64, K.ML_Q4_0, K.ML_Q8_0, 1),
                                                          (4096, 32, 8, 128, K.ML_Q8_0, K.ML_Q8_0, 0)])
def test_rmsnorm_qkv_f16_rows(dev, dim, nh, nkv, hd, typ, vtyp, bias):
    """the F16 cache's projection: the same q, and the cache row *pos holding
    the half rounding of the F32 projection's k and v (store_kv folded into
    the epilogue); no other row touched"""
    from test_gpu_kernels import rand_mat, dmat
    qd, kvd, max_seq, pos = nh * hd, nkv * hd, 40, 31
    typs = (typ, typ, vtyp)
    mats = [rand_mat(r, dim, t, 1) for r, t in zip((qd, kvd, kvd), typs)]
    Ws = [dmat(dev, q, d, dh, r, dim, t, 1) for (q, d, dh), r, t in zip(mats, (qd, kvd, kvd), typs)]
    bb = [dev.put(f32(RNG.normal(0, 0.02, r))).ptr if bias else None for r in (qd, kvd, kvd)]
    cs, sn = dev.put(f32(RNG.uniform(-1, 1, max_seq * hd // 2))), dev.put(f32(RNG.uniform(-1, 1, max_seq * hd // 2)))
    xb, wb = dev.put(f32(RNG.normal(0, 2, dim))), dev.put(f32(RNG.normal(1, 0.1, dim)))
    posb = dev.put(np.array([pos], np.int32))
    q32, k32, v32 = dev.zeros(4 * qd), dev.zeros(4 * max_seq * kvd), dev.zeros(4 * max_seq * kvd)
    K.hip.krh_rmsnorm_matvec_qkv(q32.ptr, k32.ptr, v32.ptr, *[C.byref(W) for W in Ws], *bb, xb.ptr, wb.ptr, 1e-5,
                                 cs.ptr, sn.ptr, hd, posb.ptr)
    sentinel = np.full(max_seq * kvd, 0x1234, np.uint16)
    q16, k16, v16 = dev.zeros(4 * qd), dev.put(sentinel), dev.put(sentinel)
    K.hip.krh_rmsnorm_matvec_qkv_f16(q16.ptr, k16.ptr, v16.ptr, *[C.byref(W) for W in Ws], *bb, xb.ptr, wb.ptr, 1e-5,
                                     cs.ptr, sn.ptr, hd, posb.ptr)
    ok()
    assert np.array_equal(bits(q16.get(np.float32, qd)), bits(q32.get(np.float32, qd)))
    for a32, a16 in ((k32, k16), (v32, v16)):
        want = sentinel.copy().reshape(max_seq, kvd)
        want[pos] = f16_rule(a32.get(np.float32, max_seq * kvd).reshape(max_seq, kvd)[pos])
        assert np.array_equal(a16.get(np.uint16, max_seq * kvd).reshape(max_seq, kvd), want)


@pytest.mark.parametrize("nh,nkv,hd,pos,window", [(32, 8, 128, 2175, 0), (14, 2, 64, 63, 0), (8, 2, 64, 100, 7),
                                                  (6, 6, 48, 0, 0)])
def test_attention_q8_store_folded(dev, nh, nkv, hd, pos, window):
    """decode over the Q8 cache with row *pos still in the staging rows: the
    same cache contents and output as krh_store_kv then krh_attention_kv"""
    max_seq = max(256, pos + 1)
    kvd, qd = nkv * hd, nh * hd
    q = f32(RNG.normal(0, 1, qd))
    k, v, kd, vd = rand_cache(K.ML_Q8_0, max_seq, kvd, nkv)
    krow, vrow = f32(RNG.normal(0, 1, kvd)), f32(RNG.normal(0, 2, kvd))
    krow[:hd] = 0.0   # an all-zero head: scale 0
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    posb = dev.put(np.array([pos], np.int32))
    outs = []
    for folded in (0, 1):
        kb, vb, kdb, vdb = dev.put(k), dev.put(v), dev.put(kd), dev.put(vd)
        view = K.MlKvLayer(None, None, kb.ptr, vb.ptr, kdb.ptr, vdb.ptr, window, None, None)
        ao, att = dev.zeros(4 * qd), dev.zeros(4 * nh * max_seq)
        if folded:
            K.hip.krh_attention_q8_store(ao.ptr, att.ptr, dev.put(q).ptr, C.byref(view), dev.put(krow).ptr,
                                         dev.put(vrow).ptr, nh, nkv, hd, max_seq, scale, posb.ptr)
        else:
            K.hip.krh_store_kv(K.ML_Q8_0, kb.ptr, vb.ptr, kdb.ptr, vdb.ptr, dev.put(krow).ptr, dev.put(vrow).ptr, nkv,
                               hd, posb.ptr, 1)
            K.hip.krh_attention_kv(ao.ptr, att.ptr, dev.put(q).ptr, C.byref(view), nh, nkv, hd, max_seq, scale,
                                   posb.ptr, 1, max_seq - 1)
        ok()
        outs.append([ao.get(np.float32, qd).view(np.uint32), kb.get(np.int8, max_seq * kvd), vb.get(np.int8, max_seq * kvd),
                     kdb.get(np.float32, max_seq * nkv).view(np.uint32), vdb.get(np.float32, max_seq * nkv).view(np.uint32)])
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
