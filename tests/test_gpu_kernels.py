"""Parity of each fused HIP kernel with the oracle, bit for bit, through the
C ABI of libkrafla_hip.so. Needs a gfx950 device."""
import contextlib
import ctypes as C
import os

import numpy as np
import pytest

import krafla as K
import oracle_lib as O
from oracle_lib import oracle

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(42)


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
    """device copies of numpy arrays, freed together"""

    def __init__(self):
        self.bufs = []

    def put(self, a):
        b = K.DevBuf.of(a)
        self.bufs.append(b)
        return b

    def zeros(self, nbytes):
        return self.put(np.zeros(nbytes, dtype=np.uint8))

    def free(self):
        for b in self.bufs:
            b.free()


@pytest.fixture
def dev():
    d = Dev()
    yield d
    d.free()


def test_expf_exhaustive(dev):
    """the device expf equals the host C library's on every float32 input"""
    n = 1 << 26
    xb, yb = dev.zeros(4 * n), dev.zeros(4 * n)
    bad = 0
    threads = min(16, os.cpu_count() or 1)
    for lo in range(0, 1 << 32, n):
        x = np.arange(lo, lo + n, dtype=np.uint64).astype(np.uint32).view(np.float32)
        K.check(K.hip.krh_copy_h2d(xb.ptr, x.ctypes.data, x.nbytes))
        K.hip.krh_math_batch(K.MATH_EXPF, yb.ptr, xb.ptr, None, n)
        y = yb.get(np.float32, n)
        bad += oracle.kro_expf_check_range(lo, y.ctypes.data, n, threads)
    assert bad == 0


def test_sqrt_exhaustive(dev):
    """the device square root equals the host's (IEEE, correctly rounded) on
    every non-negative float32 input"""
    n = 1 << 26
    xb, yb = dev.zeros(4 * n), dev.zeros(4 * n)
    for lo in range(0, 1 << 31, n):
        x = np.arange(lo, lo + n, dtype=np.uint64).astype(np.uint32).view(np.float32)
        K.check(K.hip.krh_copy_h2d(xb.ptr, x.ctypes.data, x.nbytes))
        K.hip.krh_math_batch(K.MATH_SQRT, yb.ptr, xb.ptr, None, n)
        y = yb.get(np.float32, n)
        want = np.sqrt(x)
        fin = ~np.isnan(want)
        assert np.array_equal(bits(y[fin]), bits(want[fin])), lo


def test_division_and_rms_inverse(dev):
    """a / b and rmsnorm's 1 / sqrtf(ss / n + eps) against numpy float32
    (IEEE round to nearest even), on random and hard operands"""
    n = 1 << 24
    a = RNG.integers(0, 0x7f800000, n, dtype=np.uint32).view(np.float32)
    b = RNG.integers(0x00800000, 0x7f800000, n, dtype=np.uint32).view(np.float32)
    a[:4096] = np.float32(1.0)
    b[:4096] = np.arange(1, 4097, dtype=np.float32)
    ab, bb, yb = dev.put(a), dev.put(b), dev.zeros(4 * n)
    K.hip.krh_math_batch(K.MATH_DIV, yb.ptr, ab.ptr, bb.ptr, n)
    with np.errstate(all="ignore"):
        want = (a / b).astype(np.float32)
    assert np.array_equal(bits(yb.get(np.float32, n)), bits(want))
    ss = f32(np.abs(RNG.normal(0, 1, n)) * RNG.choice([1e-3, 1.0, 100.0, 1e4], n))
    dn = f32(RNG.choice([48.0, 64.0, 128.0, 288.0, 896.0, 2048.0, 4096.0], n))
    sb, nb = dev.put(ss), dev.put(dn)
    K.hip.krh_math_batch(K.MATH_RMS_INV, yb.ptr, sb.ptr, nb.ptr, n)
    want = (np.float32(1.0) / np.sqrt((ss / dn).astype(np.float32) + np.float32(1e-5))).astype(np.float32)
    assert np.array_equal(bits(yb.get(np.float32, n)), bits(want))


def test_h2f_all(dev):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    hb, yb = dev.put(h), dev.zeros(4 * 65536)
    K.hip.krh_h2f_batch(yb.ptr, hb.ptr, 65536)
    y = yb.get(np.float32, 65536)
    want = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(bits(y[fin]), bits(want[fin]))
    assert np.all(np.isnan(y[np.isnan(want)]))


@pytest.mark.parametrize("n,ntok", [(32, 1), (4096, 1), (14336, 1), (288, 5)])
def test_quantize(dev, n, ntok):
    x = f32(RNG.normal(0, 1, n * ntok) * RNG.choice([1e-3, 1.0, 1e3], n * ntok))
    x[:32] = 0.0
    if n >= 96:
        x[32:64] = [1e-37 if i % 2 else -2e-37 for i in range(32)]
        x[64:96] = 0.0
        x[64:70] = [127.0, 0.5, -0.5, 1.5, 2.5, -2.5]
    if n >= 160:   # an all-NaN block (max seeded with 0: scale 0, quants 0) and a half-NaN one
        x[96:128] = np.nan
        x[128:160:2] = np.nan
    xb, qb, db = dev.put(x), dev.zeros(n * ntok), dev.zeros(4 * n * ntok // 32)
    K.hip.krh_quantize_q8(qb.ptr, db.ptr, xb.ptr, n, ntok)
    ok()
    q0, d0 = O.quantize(x)
    assert np.array_equal(qb.get(np.int8, n * ntok), q0)
    assert np.array_equal(bits(db.get(np.float32, n * ntok // 32)), bits(d0))


def rand_mat(rows, cols, typ, d16):
    if typ == K.ML_Q8_0:
        q = RNG.integers(-127, 128, rows * cols).astype(np.int8)
    else:
        q = RNG.integers(0, 256, rows * cols // 2).astype(np.uint8)
    dh = np.abs(RNG.normal(0, 0.01, rows * cols // 32)).astype(np.float16)
    d = dh.astype(np.float32) if d16 else f32(np.abs(RNG.normal(0, 0.01, rows * cols // 32)))
    return q, d, dh


def dmat(dev, q, d, dh, rows, cols, typ, d16):
    qb = dev.put(q)
    db = dev.put(dh if d16 else d)
    return K.KrhMat(qb.ptr, db.ptr, rows, cols, typ, d16)


def oracle_matvec(q, d, rows, cols, typ, xq, xd):
    W = O.qtensor(q, d, rows, cols, typ)
    y = np.zeros(rows, dtype=np.float32)
    fn = oracle.kro_matvec_q8 if typ == K.ML_Q8_0 else oracle.kro_matvec_q4
    fn(y.ctypes.data, C.byref(W), C.byref(O.qact(xq, xd)), 0, rows)
    return y


@pytest.mark.parametrize("typ", [K.ML_Q8_0, K.ML_Q4_0])
def test_block_dots_exact(dev, typ):
    rows, cols = 37, 4096
    q, d, dh = rand_mat(rows, cols, typ, 0)
    xq, xd = O.quantize(f32(RNG.normal(0, 1, cols)))
    W = dmat(dev, q, d, dh, rows, cols, typ, 0)
    sb = dev.zeros(4 * rows * cols // 32)
    K.hip.krh_block_dots(sb.ptr, C.byref(W), dev.put(xq).ptr)
    ok()
    want = np.zeros(rows * cols // 32, dtype=np.int32)
    oracle.kro_block_dots(want.ctypes.data, C.byref(O.qtensor(q, d, rows, cols, typ)), C.byref(O.qact(xq, xd)), 0,
                          rows)
    assert np.array_equal(sb.get(np.int32, rows * cols // 32), want)


MV_SHAPES = [(1, 32), (3, 96), (16, 256), (17, 288), (64, 768), (288, 768), (4096, 4096), (896, 4864),
             (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize("typ", [K.ML_Q8_0, K.ML_Q4_0])
@pytest.mark.parametrize("d16", [0, 1])
@pytest.mark.parametrize("rows,cols", MV_SHAPES)
def test_matvec(dev, typ, d16, rows, cols):
    q, d, dh = rand_mat(rows, cols, typ, d16)
    xq, xd = O.quantize(f32(RNG.normal(0, 1, cols)))
    W = dmat(dev, q, d, dh, rows, cols, typ, d16)
    yb = dev.zeros(4 * rows)
    K.hip.krh_matvec(yb.ptr, C.byref(W), dev.put(xq).ptr, dev.put(xd).ptr, 0)
    ok()
    want = oracle_matvec(q, d, rows, cols, typ, xq, xd)
    assert np.array_equal(bits(yb.get(np.float32, rows)), bits(want))


def test_matvec_accumulate(dev):
    rows, cols = 288, 768
    q, d, dh = rand_mat(rows, cols, K.ML_Q8_0, 0)
    xq, xd = O.quantize(f32(RNG.normal(0, 1, cols)))
    y0 = f32(RNG.normal(0, 1, rows))
    W = dmat(dev, q, d, dh, rows, cols, K.ML_Q8_0, 0)
    yb = dev.put(y0)
    K.hip.krh_matvec(yb.ptr, C.byref(W), dev.put(xq).ptr, dev.put(xd).ptr, 1)
    ok()
    want = (y0 + oracle_matvec(q, d, rows, cols, K.ML_Q8_0, xq, xd)).astype(np.float32)
    assert np.array_equal(bits(yb.get(np.float32, rows)), bits(want))


@pytest.mark.parametrize("n,ntok", [(288, 1), (4096, 1), (896, 3)])
def test_rmsnorm_q8(dev, n, ntok):
    x = f32(RNG.normal(0, 2, n * ntok))
    if ntok > 1:
        x[n + 5] = np.nan   # token 1: a NaN sum, every block all-NaN
    w = f32(RNG.normal(1, 0.1, n))
    qb, db, ob = dev.zeros(n * ntok), dev.zeros(4 * n * ntok // 32), dev.zeros(4 * n * ntok)
    K.hip.krh_rmsnorm_q8(qb.ptr, db.ptr, ob.ptr, dev.put(x).ptr, dev.put(w).ptr, n, 1e-5, ntok)
    ok()
    for t in range(ntok):
        o = np.zeros(n, np.float32)
        xt = f32(x[t * n:(t + 1) * n])
        oracle.kro_rmsnorm(o.ctypes.data, xt.ctypes.data, w.ctypes.data, n, C.c_float(1e-5))
        q0, d0 = O.quantize(o)
        got_o = ob.get(np.float32, n * ntok)[t * n:(t + 1) * n]
        assert np.array_equal(np.isnan(got_o), np.isnan(o))
        assert np.array_equal(bits(got_o[~np.isnan(o)]), bits(o[~np.isnan(o)]))
        assert np.array_equal(qb.get(np.int8, n * ntok)[t * n:(t + 1) * n], q0)
        assert np.array_equal(bits(db.get(np.float32, n * ntok // 32)[t * n // 32:(t + 1) * n // 32]), bits(d0))


@pytest.mark.parametrize("dim,nh,nkv,hd,typ,vtyp,bias", [(288, 6, 6, 48, K.ML_Q8_0, K.ML_Q8_0, 0),
                                                          (896, 14, 2, 64, K.ML_Q4_0, K.ML_Q8_0, 1),
                                                          (896, 14, 2, 64, K.ML_Q4_0, K.ML_Q4_0, 1),
                                                          (2048, 32, 8, 64, K.ML_Q4_0, K.ML_Q8_0, 0),
                                                          (4096, 32, 8, 128, K.ML_Q8_0, K.ML_Q8_0, 0)])
def test_qkv_bias_rope_cache(dev, dim, nh, nkv, hd, typ, vtyp, bias):
    qd, kvd, max_seq, pos = nh * hd, nkv * hd, 40, 23
    typs = (typ, typ, vtyp)
    mats = [rand_mat(r, dim, t, 1) for r, t in zip((qd, kvd, kvd), typs)]
    Ws = [dmat(dev, q, d, dh, r, dim, t, 1) for (q, d, dh), r, t in zip(mats, (qd, kvd, kvd), typs)]
    biases = [f32(RNG.normal(0, 0.02, r)) for r in (qd, kvd, kvd)]
    cs, sn = f32(RNG.uniform(-1, 1, max_seq * hd // 2)), f32(RNG.uniform(-1, 1, max_seq * hd // 2))
    xq, xd = O.quantize(f32(RNG.normal(0, 1, dim)))
    qb, kc, vc = dev.zeros(4 * qd), dev.zeros(4 * max_seq * kvd), dev.zeros(4 * max_seq * kvd)
    bb = [dev.put(b) if bias else None for b in biases]
    posb = dev.put(np.array([pos], np.int32))
    K.hip.krh_matvec_qkv(qb.ptr, kc.ptr, vc.ptr, C.byref(Ws[0]), C.byref(Ws[1]), C.byref(Ws[2]),
                         *[b.ptr if b else None for b in bb], dev.put(xq).ptr, dev.put(xd).ptr,
                         dev.put(cs).ptr, dev.put(sn).ptr, hd, posb.ptr)
    ok()
    outs = []
    for (q, d, dh), r, b, t in zip(mats, (qd, kvd, kvd), biases, typs):
        y = oracle_matvec(q, d, r, dim, t, xq, xd)
        if bias:
            oracle.kro_add(y.ctypes.data, b.ctypes.data, r)
        outs.append(y)
    c0 = f32(cs[pos * hd // 2:(pos + 1) * hd // 2])
    s0 = f32(sn[pos * hd // 2:(pos + 1) * hd // 2])
    oracle.kro_rope(outs[0].ctypes.data, outs[1].ctypes.data, c0.ctypes.data, s0.ctypes.data, hd, nh, nkv)
    assert np.array_equal(bits(qb.get(np.float32, qd)), bits(outs[0]))
    assert np.array_equal(bits(kc.get(np.float32, max_seq * kvd)[pos * kvd:(pos + 1) * kvd]), bits(outs[1]))
    assert np.array_equal(bits(vc.get(np.float32, max_seq * kvd)[pos * kvd:(pos + 1) * kvd]), bits(outs[2]))


@pytest.mark.parametrize("rows,cols,typ", [(768, 288, K.ML_Q8_0), (4864, 896, K.ML_Q4_0), (14336, 4096, K.ML_Q8_0),
                                           (8192, 2048, K.ML_Q4_0), (40, 96, K.ML_Q8_0)])
def test_swiglu(dev, rows, cols, typ):
    (q1, d1, h1), (q3, d3, h3) = rand_mat(rows, cols, typ, 1), rand_mat(rows, cols, typ, 1)
    W1, W3 = dmat(dev, q1, d1, h1, rows, cols, typ, 1), dmat(dev, q3, d3, h3, rows, cols, typ, 1)
    xq, xd = O.quantize(f32(RNG.normal(0, 1, cols) * 30))
    hb = dev.zeros(4 * rows)
    K.hip.krh_matvec_swiglu(hb.ptr, C.byref(W1), C.byref(W3), dev.put(xq).ptr, dev.put(xd).ptr)
    ok()
    g = oracle_matvec(q1, d1, rows, cols, typ, xq, xd)
    u = oracle_matvec(q3, d3, rows, cols, typ, xq, xd)
    oracle.kro_silu_mul(g.ctypes.data, u.ctypes.data, rows)
    assert np.array_equal(bits(hb.get(np.float32, rows)), bits(g))


@pytest.mark.parametrize("typ,d16", [(K.ML_Q8_0, 1), (K.ML_Q4_0, 0)])
@pytest.mark.parametrize("rows,cols", [(4096, 14336), (4096, 4096), (896, 4864), (288, 768), (5, 64)])
def test_matvec_float_input(dev, typ, d16, rows, cols):
    """y += W quantize_q8(x): the input quantized inside the launch, as
    transformer.c quantizes hb and ao before w2 and wo"""
    q, d, dh = rand_mat(rows, cols, typ, d16)
    x = f32(RNG.normal(0, 1, cols) * RNG.choice([1e-3, 1.0, 50.0], cols))
    x[:32] = 0.0
    y0 = f32(RNG.normal(0, 1, rows))
    W = dmat(dev, q, d, dh, rows, cols, typ, d16)
    yb = dev.put(y0)
    K.hip.krh_matvec_f(yb.ptr, C.byref(W), dev.put(x).ptr, 1)
    ok()
    xq, xd = O.quantize(x)
    want = (y0 + oracle_matvec(q, d, rows, cols, typ, xq, xd)).astype(np.float32)
    assert np.array_equal(bits(yb.get(np.float32, rows)), bits(want))


@pytest.mark.parametrize("nh,nkv,hd,pos,window", [(6, 6, 48, 0, 0), (6, 6, 48, 200, 0), (14, 2, 64, 511, 0),
                                                    (32, 8, 128, 2175, 0), (32, 8, 128, 2174, 0),
                                                  (32, 8, 128, 2303, 0), (32, 8, 64, 4000, 0), (8, 2, 64, 100, 7),
                                                  (16, 1, 64, 63, 0), (4, 2, 32, 64, 0), (12, 4, 96, 130, 0),
                                                  (4, 2, 32, 9000, 0), (8, 2, 64, 12000, 9000), (8, 4, 256, 300, 0),
                                                  (4, 1, 256, 200, 64),
                                                  # the softmax inside the mix launch (rows of at most 4096
                                                  # scores, groups of 1 to 4): at the limit, groups 1 and 2
                                                  (32, 8, 128, 4095, 0), (8, 8, 64, 1000, 0), (8, 4, 64, 3000, 0),
                                                  (6, 3, 64, 4095, 100)])
def test_attention(dev, nh, nkv, hd, pos, window):
    max_seq = max(256, pos + 1)
    kvd, qd = nkv * hd, nh * hd
    q = f32(RNG.normal(0, 1, qd))
    kc = f32(RNG.normal(0, 1, max_seq * kvd))
    vc = f32(RNG.normal(0, 1, max_seq * kvd))
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    ao, aq, ad, att = dev.zeros(4 * qd), dev.zeros(qd), dev.zeros(4 * qd // 32), dev.zeros(4 * nh * max_seq)
    posb = dev.put(np.array([pos], np.int32))
    K.hip.krh_attention(ao.ptr, aq.ptr, ad.ptr, att.ptr, dev.put(q).ptr, dev.put(kc).ptr, dev.put(vc).ptr, nh, nkv,
                        hd, max_seq, window, float(scale), posb.ptr)
    ok()
    cfg = K.MlConfig(n_heads=nh, n_kv_heads=nkv, head_dim=hd, kv_dim=kvd, q_dim=qd, max_seq=max_seq,
                     attn_scale=float(scale))
    kvl = O.KvLayer(kc.ctypes.data, vc.ctypes.data, None, None, None, None, window, None, None)
    out = np.zeros(qd, np.float32)
    scratch = np.zeros(max_seq, np.float32)
    oracle.kro_attention(out.ctypes.data, q.ctypes.data, C.byref(kvl), scratch.ctypes.data, C.byref(cfg), pos)
    assert np.array_equal(bits(ao.get(np.float32, qd)), bits(out))
    q0, d0 = O.quantize(out)
    assert np.array_equal(aq.get(np.int8, qd), q0)
    assert np.array_equal(bits(ad.get(np.float32, qd // 32)), bits(d0))


def seq_sum_f32(t, s0=0.0):
    """((s0 + t0) + t1) + ... in float32, one rounding per add (the reference's
    loop order, kernels/scalar/k_scalar.c:61, :71-74)"""
    return np.add.accumulate(np.concatenate([[np.float32(s0)], t]).astype(np.float32), dtype=np.float32)[-1]


def test_seq_sum_f32_is_sequential():
    t = f32(RNG.normal(0, 1, 300) ** 2)
    s = np.float32(0)
    for v in t:
        s = np.float32(s + v)
    assert bits(np.float32(seq_sum_f32(t))) == bits(s)


ORDERED_CASES = ["squares", "heavy", "outliers", "absorb", "absorb_late", "tiny", "zeros", "exps", "mixed_sign",
                 "nan", "inf", "huge", "ties", "steep", "late_growth", "neg_zero", "subnormal"]


def ordered_terms(case, n):
    """the terms of one ordered-sum case"""
    x = RNG.normal(0, 1, n)
    if case == "squares":
        t = f32(x) * f32(x)
    elif case == "heavy":
        t = f32(x / np.sqrt(np.abs(RNG.normal(0, 1, n)) + 0.05)) ** 2
    elif case == "outliers":
        x[RNG.random(n) < 0.01] *= 80
        t = f32(x) ** 2
    elif case == "absorb":
        t = f32(np.ones(n))
        t[0] = 1e8
    elif case == "absorb_late":
        t = f32(np.full(n, 0.75))
        t[n // 3] = 3e7
    elif case == "tiny":
        t = f32(np.abs(x) * 1e-41)
    elif case == "zeros":
        t = f32(np.zeros(n))
    elif case == "exps":
        t = f32(np.exp(-8 * RNG.random(n)))
    elif case == "mixed_sign":
        t = f32(x * 100)
    elif case == "nan":
        t = f32(x * x)
        t[n // 2] = np.nan
    elif case == "inf":
        t = f32(x * x)
        t[n - 1] = np.inf
    elif case == "ties":   # few significant bits: rounding ties all along
        t = f32(RNG.integers(0, 8, n)) * f32(2.0) ** f32(RNG.integers(-3, 4, n))
    elif case == "steep":   # the running sum doubles every few terms
        t = f32(2.0) ** f32(np.floor(np.arange(n) * 60.0 / max(n, 1)) - 30)
    elif case == "late_growth":
        t = f32(x * x)
        t[: n // 2] = 0
    elif case == "neg_zero":
        t = f32(x * x)
        t[RNG.random(n) < 0.05] = -0.0
    elif case == "subnormal":
        t = f32(np.abs(x) * 1e-44)
    else:   # huge: the sum overflows to inf part-way
        t = f32(np.full(n, 3e37))
    return f32(t)


@pytest.mark.parametrize("s0", [0.0, 1234.5678])
@pytest.mark.parametrize("case", ORDERED_CASES)
@pytest.mark.parametrize("n", [1, 5, 31, 32, 33, 127, 128, 129, 2048, 2049, 2175, 4096, 4097, 8192])
def test_ordered_sum(dev, case, n, s0):
    """the chunked sum returns the bits of the sequential fp32 sum through its
    shifted runs (ties to even included), its blocks where the running sum
    changes binade (many of them for steep growth), its per-run fallback, the
    sequential path for negative, -0 and non-finite terms, and sizes at the
    chunk-length and chunk-count edges"""
    t = ordered_terms(case, n)
    out = dev.zeros(4)
    K.hip.krh_ordered_sum(out.ptr, dev.put(t).ptr, n, s0)
    ok()
    got = out.get(np.float32, 1)[0]
    want = seq_sum_f32(t, s0)
    if np.isnan(want):
        assert np.isnan(got)
    else:
        assert bits(np.float32(got)) == bits(np.float32(want)), (got, want)


@pytest.mark.parametrize("s0", [0.0, 1234.5678])
@pytest.mark.parametrize("case", ORDERED_CASES)
@pytest.mark.parametrize("n", [1, 5, 31, 33, 128, 129, 2047, 2048, 2049, 4096, 4097, 8192])
def test_ordered_sum_1024(dev, case, n, s0):
    """the ordered sum by a workgroup of 1024 threads (16 waves: the decode
    softmax's form, k_attn_softmax): the sequential fp32 sum's bits on every
    case"""
    t = ordered_terms(case, n)
    out = dev.zeros(4)
    K.hip.krh_ordered_sum_1024(out.ptr, dev.put(t).ptr, n, s0)
    ok()
    got = out.get(np.float32, 1)[0]
    want = seq_sum_f32(t, s0)
    if np.isnan(want):
        assert np.isnan(got)
    else:
        assert bits(np.float32(got)) == bits(np.float32(want)), (got, want)


@pytest.mark.parametrize("s0", [0.0, 1234.5678])
@pytest.mark.parametrize("case", ORDERED_CASES)
@pytest.mark.parametrize("n", [1, 5, 31, 33, 128, 129, 2047, 2048, 2049, 3000, 4096, 4097, 8192])
def test_ordered_sum_lean(dev, case, n, s0):
    """the ordered sum with fewer reads in flight (one chain block read
    ahead, estimates 4 reads at a time: the long-row prefill softmax's form):
    the sequential fp32 sum's bits on every case"""
    t = ordered_terms(case, n)
    out = dev.zeros(4)
    K.hip.krh_ordered_sum_lean(out.ptr, dev.put(t).ptr, n, s0)
    ok()
    got = out.get(np.float32, 1)[0]
    want = seq_sum_f32(t, s0)
    if np.isnan(want):
        assert np.isnan(got)
    else:
        assert bits(np.float32(got)) == bits(np.float32(want)), (got, want)


@pytest.mark.parametrize("s0", [0.0, 1234.5678])
@pytest.mark.parametrize("case", ORDERED_CASES)
@pytest.mark.parametrize("n", [1, 5, 31, 32, 33, 127, 128, 129, 2047, 2048, 2049, 4095, 4096])
def test_ordered_sum_wave(dev, case, n, s0):
    """the single-wave mode of the ordered sum (the batched softmax's), run by
    a workgroup's second wave: the sequential fp32 sum's bits on every case"""
    t = ordered_terms(case, n)
    out = dev.zeros(4)
    K.hip.krh_ordered_sum_wave(out.ptr, dev.put(t).ptr, n, s0)
    ok()
    got = out.get(np.float32, 1)[0]
    want = seq_sum_f32(t, s0)
    if np.isnan(want):
        assert np.isnan(got)
    else:
        assert bits(np.float32(got)) == bits(np.float32(want)), (got, want)


@pytest.mark.parametrize("case", ["random", "ties", "neg_inf", "nan0", "nans", "signed_zero", "tail_max", "all_nan"])
@pytest.mark.parametrize("n", [151936, 128256, 32003, 4097, 5, 3, 1])
def test_argmax(dev, case, n):
    """model/sampler.c:57-61 on the device: first index of the maximum, NaNs
    skipped, 0 when v[0] is NaN; repeated calls (the partials counter is
    reset by the kernel itself)"""
    v = f32(RNG.normal(0, 1, n))
    if case == "ties":
        v[:] = 0
        for i in (40000, 9, 150000, n - 1):
            if i < n:
                v[i] = 3.0
    elif case == "neg_inf":
        v[:] = -np.inf
    elif case == "nan0":
        v[0] = np.nan
    elif case == "nans":
        v[RNG.integers(0, n, max(1, n // 7))] = np.nan
        v[0] = 1.0
    elif case == "signed_zero":
        v[:] = -1.0
        v[n // 2] = -0.0
        v[n - 1] = 0.0
    elif case == "tail_max":
        v[n - 1] = 50.0
    elif case == "all_nan":
        v[:] = np.nan
    want = oracle.kro_argmax(v.ctypes.data, n)
    vb = dev.put(v)
    for rep in range(3):
        tb, pb, lb = dev.zeros(4), dev.put(np.array([5 + rep], np.int32)), dev.zeros(4 * 16)
        K.hip.krh_argmax(tb.ptr, vb.ptr, n, pb.ptr, lb.ptr)
        ok()
        assert tb.get(np.int32, 1)[0] == want
        assert pb.get(np.int32, 1)[0] == 6 + rep and lb.get(np.int32, 16)[6 + rep] == want


@pytest.mark.parametrize("typ,d16,scale", [(K.ML_Q8_0, 0, 1.0), (K.ML_Q4_0, 1, 1.0), (K.ML_Q8_0, 1, 8.0)])
def test_embed(dev, typ, d16, scale):
    rows, cols = 50, 896
    q, d, dh = rand_mat(rows, cols, typ, d16)
    E = dmat(dev, q, d, dh, rows, cols, typ, d16)
    xb = dev.zeros(4 * cols)
    K.hip.krh_embed(xb.ptr, C.byref(E), dev.put(np.array([33], np.int32)).ptr, scale)
    ok()
    want = np.zeros(cols, np.float32)
    oracle.kro_dequant_row(want.ctypes.data, C.byref(O.qtensor(q, d, rows, cols, typ)), 33)
    if scale != 1.0:
        want = (want * np.float32(scale)).astype(np.float32)
    assert np.array_equal(bits(xb.get(np.float32, cols)), bits(want))


# ---- batched prefill ----

def transposed_scales(dq, T, nb, ldx):
    """[T][nb] scales -> [nb][ldx] (the layout krh_matmul reads)"""
    out = np.zeros((nb, ldx), np.float32)
    out[:, :T] = dq.reshape(T, nb).T
    return out


@pytest.mark.parametrize("typ,d16", [(K.ML_Q8_0, 1), (K.ML_Q4_0, 1), (K.ML_Q8_0, 0), (K.ML_Q4_0, 0)])
@pytest.mark.parametrize("rows,cols,T", [(100, 64, 37), (256, 288, 130), (896, 4864, 5), (4096, 4096, 129),
                                         (1024, 14336, 64), (33, 32, 1)])
def test_matmul(dev, typ, d16, rows, cols, T):
    """int8-MFMA matmul: every token's row equals the matvec's, bit for bit
    (the reference's matmul column == matvec rule, tests/test_kernels.c:146-189)"""
    q, d, dh = rand_mat(rows, cols, typ, d16)
    X = f32(RNG.normal(0, 1, (T, cols)) * RNG.choice([1e-2, 1.0, 30.0], (T, 1)))
    ldx = (T + 127) // 128 * 128
    xq = np.zeros((ldx, cols), np.int8)
    xd = np.zeros((T, cols // 32), np.float32)
    for t in range(T):
        xq[t], xd[t] = O.quantize(X[t])
    W = dmat(dev, q, d, dh, rows, cols, typ, d16)
    y0 = f32(RNG.normal(0, 1, (T, rows)))
    for acc in (0, 1):
        yb = dev.put(y0)
        K.hip.krh_matmul(yb.ptr, rows, C.byref(W), dev.put(xq).ptr,
                         dev.put(transposed_scales(xd, T, cols // 32, ldx)).ptr, ldx, T, acc)
        ok()
        got = yb.get(np.float32, T * rows).reshape(T, rows)
        # the same product over the scales in token rows, sized exactly [T][nb]
        yr = dev.put(y0)
        K.hip.krh_matmul_rows(yr.ptr, rows, C.byref(W), dev.put(xq).ptr, dev.put(xd).ptr, ldx, T, acc)
        ok()
        got_rows = yr.get(np.float32, T * rows).reshape(T, rows)
        for t in range(T):
            want = oracle_matvec(q, d, rows, cols, typ, xq[t], xd[t])
            if acc:
                want = (y0[t] + want).astype(np.float32)
            assert np.array_equal(bits(got[t]), bits(want)), (t, acc)
            assert np.array_equal(bits(got_rows[t]), bits(want)), (t, acc, "rows")


@pytest.mark.parametrize("dim,nh,nkv,hd,typ,vtyp,bias", [(288, 6, 6, 48, K.ML_Q8_0, K.ML_Q8_0, 0),
                                                          (896, 14, 2, 64, K.ML_Q4_0, K.ML_Q8_0, 1),
                                                          (4096, 32, 8, 128, K.ML_Q8_0, K.ML_Q8_0, 0)])
def test_matmul_qkv_matches_decode(dev, dim, nh, nkv, hd, typ, vtyp, bias):
    """the batched projections (bias, RoPE, cache rows) equal the decode
    step's for every token"""
    qd, kvd, max_seq, pos0, T = nh * hd, nkv * hd, 300, 17, 140
    typs = (typ, typ, vtyp)
    mats = [rand_mat(r, dim, t, 1) for r, t in zip((qd, kvd, kvd), typs)]
    Ws = [dmat(dev, q, d, dh, r, dim, t, 1) for (q, d, dh), r, t in zip(mats, (qd, kvd, kvd), typs)]
    bb = [dev.put(f32(RNG.normal(0, 0.02, r))) if bias else None for r in (qd, kvd, kvd)]
    cs, sn = dev.put(f32(RNG.uniform(-1, 1, max_seq * hd // 2))), dev.put(f32(RNG.uniform(-1, 1, max_seq * hd // 2)))
    ldx = (T + 127) // 128 * 128
    xq = np.zeros((ldx, dim), np.int8)
    xd = np.zeros((T, dim // 32), np.float32)
    for t in range(T):
        xq[t], xd[t] = O.quantize(f32(RNG.normal(0, 1, dim)))
    qb, kc, vc = dev.zeros(4 * T * qd), dev.zeros(4 * max_seq * kvd), dev.zeros(4 * max_seq * kvd)
    K.hip.krh_matmul_qkv(qb.ptr, kc.ptr, vc.ptr, C.byref(Ws[0]), C.byref(Ws[1]), C.byref(Ws[2]),
                         *[b.ptr if b else None for b in bb], dev.put(xq).ptr,
                         dev.put(transposed_scales(xd, T, dim // 32, ldx)).ptr, ldx, T, cs.ptr, sn.ptr, hd, pos0)
    ok()
    got_q = qb.get(np.float32, T * qd).reshape(T, qd)
    got_k = kc.get(np.float32, max_seq * kvd).reshape(max_seq, kvd)
    got_v = vc.get(np.float32, max_seq * kvd).reshape(max_seq, kvd)
    q1, k1, v1 = dev.zeros(4 * qd), dev.zeros(4 * max_seq * kvd), dev.zeros(4 * max_seq * kvd)
    for t in range(0, T, 13):
        posb = dev.put(np.array([pos0 + t], np.int32))
        K.hip.krh_matvec_qkv(q1.ptr, k1.ptr, v1.ptr, C.byref(Ws[0]), C.byref(Ws[1]), C.byref(Ws[2]),
                             *[b.ptr if b else None for b in bb], dev.put(xq[t]).ptr, dev.put(xd[t]).ptr,
                             cs.ptr, sn.ptr, hd, posb.ptr)
        ok()
        p = pos0 + t
        assert np.array_equal(bits(got_q[t]), bits(q1.get(np.float32, qd)))
        assert np.array_equal(bits(got_k[p]), bits(k1.get(np.float32, max_seq * kvd)[p * kvd:(p + 1) * kvd]))
        assert np.array_equal(bits(got_v[p]), bits(v1.get(np.float32, max_seq * kvd)[p * kvd:(p + 1) * kvd]))


@pytest.mark.parametrize("nh,nkv,hd,pos0,T,window", [(6, 6, 48, 0, 40, 0), (32, 8, 128, 100, 70, 0),
                                                     (14, 2, 64, 3, 200, 0), (8, 2, 64, 10, 50, 7),
                                                     (8, 4, 256, 5, 40, 0), (4, 1, 256, 100, 30, 64),
                                                     # the MFMA kernels' groups 1, 2, 4 (4, 2, 1 row
                                                     # blocks a workgroup), the last ending at row 511
                                                     (8, 8, 64, 37, 90, 0), (16, 8, 128, 0, 33, 0),
                                                     (32, 8, 64, 5, 100, 0), (8, 4, 64, 450, 62, 0)])
@pytest.mark.parametrize("rb", [False, True])
def test_attention_batch_matches_decode(dev, nh, nkv, hd, pos0, T, window, rb):
    """rb: the register-blocked kernels forced on (64- and 128-dim heads; at
    these sizes the launch would take the per-token-block kernels)"""
    if rb and hd not in (64, 128):
        pytest.skip("the register-blocked kernels take 64- and 128-dim heads")
    with rb_forced(rb):
        attention_batch_case(dev, nh, nkv, hd, pos0, T, window)


@contextlib.contextmanager
def rb_forced(on):
    """the register-blocked prefill attention kernels for any size while on"""
    if on:
        K.hip.krh_set_attn_rb_min(0)
    try:
        yield
    finally:
        K.hip.krh_set_attn_rb_min(512)


def attention_batch_case(dev, nh, nkv, hd, pos0, T, window):
    max_seq = 512
    kvd, qd = nkv * hd, nh * hd
    Q = f32(RNG.normal(0, 1, (T, qd)))
    kc = f32(RNG.normal(0, 1, max_seq * kvd))
    vc = f32(RNG.normal(0, 1, max_seq * kvd))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    kb, vb = dev.put(kc), dev.put(vc)
    ao, att = dev.zeros(4 * T * qd), dev.zeros(4 * T * nh * max_seq)
    K.hip.krh_attention_batch(ao.ptr, att.ptr, dev.put(Q).ptr, kb.ptr, vb.ptr, nh, nkv, hd, max_seq, window, scale,
                              dev.put(np.array([pos0], np.int32)).ptr, T, pos0 + T - 1)
    ok()
    got = ao.get(np.float32, T * qd).reshape(T, qd)
    cfg = K.MlConfig(n_heads=nh, n_kv_heads=nkv, head_dim=hd, kv_dim=kvd, q_dim=qd, max_seq=max_seq,
                     attn_scale=scale)
    kvl = O.KvLayer(kc.ctypes.data, vc.ctypes.data, None, None, None, None, window, None, None)
    scratch = np.zeros(max_seq, np.float32)
    for t in range(T):
        out = np.zeros(qd, np.float32)
        qt = f32(Q[t])
        oracle.kro_attention(out.ctypes.data, qt.ctypes.data, C.byref(kvl), scratch.ctypes.data, C.byref(cfg),
                             pos0 + t)
        assert np.array_equal(bits(got[t]), bits(out)), t


@pytest.mark.parametrize("nh,nkv,hd", [(32, 8, 128), (8, 8, 64), (16, 8, 64)])
@pytest.mark.parametrize("rb", [False, True])
def test_attention_batch_stale_rows(dev, nh, nkv, hd, rb):
    """cache rows past the last token's position and score rows past each
    token's own position hold NaN (rows still to be written, stale scores):
    the batched attention lets none of them reach a result (both kernel
    choices)"""
    with rb_forced(rb):
        stale_rows_case(dev, nh, nkv, hd)


def stale_rows_case(dev, nh, nkv, hd):
    max_seq, pos0, T = 512, 40, 75
    kvd, qd = nkv * hd, nh * hd
    Q = f32(RNG.normal(0, 1, (T, qd)))
    kc = f32(RNG.normal(0, 1, max_seq * kvd))
    vc = f32(RNG.normal(0, 1, max_seq * kvd))
    kc[(pos0 + T) * kvd:] = np.nan
    vc[(pos0 + T) * kvd:] = np.nan
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    ao, att = dev.zeros(4 * T * qd), dev.put(np.full(T * nh * max_seq, np.nan, np.float32))
    K.hip.krh_attention_batch(ao.ptr, att.ptr, dev.put(Q).ptr, dev.put(kc).ptr, dev.put(vc).ptr, nh, nkv, hd,
                              max_seq, 0, scale, dev.put(np.array([pos0], np.int32)).ptr, T, pos0 + T - 1)
    ok()
    got = ao.get(np.float32, T * qd).reshape(T, qd)
    assert not np.isnan(got).any()
    cfg = K.MlConfig(n_heads=nh, n_kv_heads=nkv, head_dim=hd, kv_dim=kvd, q_dim=qd, max_seq=max_seq,
                     attn_scale=scale)
    kvl = O.KvLayer(kc.ctypes.data, vc.ctypes.data, None, None, None, None, 0, None, None)
    scratch = np.zeros(max_seq, np.float32)
    for t in range(T):
        out = np.zeros(qd, np.float32)
        qt = f32(Q[t])
        oracle.kro_attention(out.ctypes.data, qt.ctypes.data, C.byref(kvl), scratch.ctypes.data, C.byref(cfg),
                             pos0 + t)
        assert np.array_equal(bits(got[t]), bits(out)), t


def test_silu_quant(dev):
    n, T = 4864, 9
    g, u = f32(RNG.normal(0, 3, (T, n))), f32(RNG.normal(0, 1, (T, n)))
    g[2, :32] = np.nan   # an all-NaN block
    u[3, 40] = np.nan    # one NaN in a block
    ldx = 128
    qb, db = dev.zeros(T * n), dev.zeros(4 * (n // 32) * ldx)
    K.hip.krh_silu_quant(qb.ptr, db.ptr, ldx, dev.put(g).ptr, dev.put(u).ptr, n, T)
    ok()
    q = qb.get(np.int8, T * n).reshape(T, n)
    d = db.get(np.float32, (n // 32) * ldx).reshape(n // 32, ldx)
    for t in range(T):
        h = f32(g[t])
        oracle.kro_silu_mul(h.ctypes.data, f32(u[t]).ctypes.data, n)
        q0, d0 = O.quantize(h)
        assert np.array_equal(q[t], q0) and np.array_equal(bits(d[:, t]), bits(d0))


@pytest.mark.parametrize("typ,d16", [(K.ML_Q8_0, 1), (K.ML_Q4_0, 1), (K.ML_Q8_0, 0)])
@pytest.mark.parametrize("rows,cols,T", [(14336, 4096, 300), (4864, 896, 511), (768, 288, 37), (96, 64, 5),
                                         (8192, 2048, 129)])
def test_matmul_swiglu_matches_separate(dev, typ, d16, rows, cols, T):
    """krh_matmul_swiglu (w1 and w3 tiles in one launch, SiLU and the Q8_0 of
    h in its epilogue) gives the bits of two krh_matmul calls and
    krh_silu_quant (both pinned to the oracle above): the quants and the
    transposed scales of every token (96 rows: a half-empty last tile)"""
    mats = [rand_mat(rows, cols, typ, d16) for _ in range(2)]
    Ws = [dmat(dev, q, d, dh, rows, cols, typ, d16) for q, d, dh in mats]
    X = f32(RNG.normal(0, 1, (T, cols)) * RNG.choice([1e-2, 1.0, 30.0], (T, 1)))
    ldx = (T + 127) // 128 * 128
    xq = np.zeros((ldx, cols), np.int8)
    xd = np.zeros((T, cols // 32), np.float32)
    for t in range(T):
        xq[t], xd[t] = O.quantize(X[t])
    xqb, xdb = dev.put(xq), dev.put(transposed_scales(xd, T, cols // 32, ldx))
    g, u = dev.zeros(4 * ldx * rows), dev.zeros(4 * ldx * rows)
    K.hip.krh_matmul(g.ptr, rows, C.byref(Ws[0]), xqb.ptr, xdb.ptr, ldx, T, 0)
    K.hip.krh_matmul(u.ptr, rows, C.byref(Ws[1]), xqb.ptr, xdb.ptr, ldx, T, 0)
    wq, wd = dev.zeros(ldx * rows), dev.zeros(4 * ldx * rows // 32)
    K.hip.krh_silu_quant(wq.ptr, wd.ptr, ldx, g.ptr, u.ptr, rows, T)
    hq, hd = dev.zeros(ldx * rows), dev.zeros(4 * ldx * rows // 32)
    K.hip.krh_matmul_swiglu(hq.ptr, hd.ptr, C.byref(Ws[0]), C.byref(Ws[1]), xqb.ptr, xdb.ptr, ldx, T)
    ok()
    assert np.array_equal(hq.get(np.int8, ldx * rows).reshape(ldx, rows)[:T],
                          wq.get(np.int8, ldx * rows).reshape(ldx, rows)[:T])
    got_d = hd.get(np.float32, ldx * rows // 32).reshape(rows // 32, ldx)[:, :T]
    want_d = wd.get(np.float32, ldx * rows // 32).reshape(rows // 32, ldx)[:, :T]
    assert np.array_equal(bits(got_d), bits(want_d))


def test_matmul_swiglu_rejects_mismatched_pairs(dev):
    q, d, dh = rand_mat(64, 64, K.ML_Q8_0, 1)
    W1 = dmat(dev, q, d, dh, 64, 64, K.ML_Q8_0, 1)
    W3 = dmat(dev, q, d, dh, 64, 64, K.ML_Q8_0, 0)   # another scale width
    buf = dev.zeros(4 * 128 * 64)
    K.hip.krh_matmul_swiglu(buf.ptr, buf.ptr, C.byref(W1), C.byref(W3), buf.ptr, buf.ptr, 128, 5)
    assert K.hip.krh_status() == K.ML_E_SHAPE
    K.hip.krh_clear_error()


# ---- rmsnorm fused into the consuming matvec ----

def oracle_norm_q8(x, w, eps=1e-5):
    o = np.zeros(len(x), np.float32)
    oracle.kro_rmsnorm(o.ctypes.data, f32(x).ctypes.data, f32(w).ctypes.data, len(x), C.c_float(eps))
    return O.quantize(o)


@pytest.mark.parametrize("typ,d16", [(K.ML_Q8_0, 1), (K.ML_Q4_0, 0)])
@pytest.mark.parametrize("rows,cols", [(32000, 288), (4096, 4096), (5000, 2048), (7, 64)])
def test_rmsnorm_matvec(dev, typ, d16, rows, cols):
    """the classifier launch: rmsnorm, quantize, matvec (model/transformer.c:299-303);
    more row tiles than workgroups, so workgroups loop"""
    q, d, dh = rand_mat(rows, cols, typ, d16)
    x = f32(RNG.normal(0, 3, cols))
    w = f32(RNG.normal(1, 0.1, cols))
    W = dmat(dev, q, d, dh, rows, cols, typ, d16)
    yb = dev.zeros(4 * rows)
    K.hip.krh_rmsnorm_matvec(yb.ptr, C.byref(W), dev.put(x).ptr, dev.put(w).ptr, 1e-5, 0)
    ok()
    xq, xd = oracle_norm_q8(x, w)
    assert np.array_equal(bits(yb.get(np.float32, rows)), bits(oracle_matvec(q, d, rows, cols, typ, xq, xd)))


@pytest.mark.parametrize("dim,nh,nkv,hd,typ,vtyp,bias", [(896, 14, 2, 64, K.ML_Q4_0, K.ML_Q8_0, 1),
                                                          (4096, 32, 8, 128, K.ML_Q8_0, K.ML_Q8_0, 0)])
def test_rmsnorm_qkv_matches_unfused(dev, dim, nh, nkv, hd, typ, vtyp, bias):
    qd, kvd, max_seq, pos = nh * hd, nkv * hd, 40, 31
    typs = (typ, typ, vtyp)
    mats = [rand_mat(r, dim, t, 1) for r, t in zip((qd, kvd, kvd), typs)]
    Ws = [dmat(dev, q, d, dh, r, dim, t, 1) for (q, d, dh), r, t in zip(mats, (qd, kvd, kvd), typs)]
    bb = [dev.put(f32(RNG.normal(0, 0.02, r))).ptr if bias else None for r in (qd, kvd, kvd)]
    cs, sn = dev.put(f32(RNG.uniform(-1, 1, max_seq * hd // 2))), dev.put(f32(RNG.uniform(-1, 1, max_seq * hd // 2)))
    x, w = f32(RNG.normal(0, 2, dim)), f32(RNG.normal(1, 0.1, dim))
    posb = dev.put(np.array([pos], np.int32))
    outs = []
    for fused in (1, 0):
        qb, kc, vc = dev.zeros(4 * qd), dev.zeros(4 * max_seq * kvd), dev.zeros(4 * max_seq * kvd)
        if fused:
            K.hip.krh_rmsnorm_matvec_qkv(qb.ptr, kc.ptr, vc.ptr, *[C.byref(W) for W in Ws], *bb, dev.put(x).ptr,
                                         dev.put(w).ptr, 1e-5, cs.ptr, sn.ptr, hd, posb.ptr)
        else:
            xq, xd = oracle_norm_q8(x, w)
            K.hip.krh_matvec_qkv(qb.ptr, kc.ptr, vc.ptr, *[C.byref(W) for W in Ws], *bb, dev.put(xq).ptr,
                                 dev.put(xd).ptr, cs.ptr, sn.ptr, hd, posb.ptr)
        ok()
        outs.append([b.get(np.float32, n) for b, n in ((qb, qd), (kc, max_seq * kvd), (vc, max_seq * kvd))])
    for a, b in zip(*outs):
        assert np.array_equal(bits(a), bits(b))


@pytest.mark.parametrize("rows,cols,typ", [(14336, 4096, K.ML_Q8_0), (4864, 896, K.ML_Q4_0)])
def test_rmsnorm_swiglu(dev, rows, cols, typ):
    (q1, d1, h1), (q3, d3, h3) = rand_mat(rows, cols, typ, 1), rand_mat(rows, cols, typ, 1)
    W1, W3 = dmat(dev, q1, d1, h1, rows, cols, typ, 1), dmat(dev, q3, d3, h3, rows, cols, typ, 1)
    x, w = f32(RNG.normal(0, 2, cols)), f32(RNG.normal(1, 0.1, cols))
    hb = dev.zeros(4 * rows)
    K.hip.krh_rmsnorm_matvec_swiglu(hb.ptr, C.byref(W1), C.byref(W3), dev.put(x).ptr, dev.put(w).ptr, 1e-5)
    ok()
    xq, xd = oracle_norm_q8(x, w)
    g = oracle_matvec(q1, d1, rows, cols, typ, xq, xd)
    u = oracle_matvec(q3, d3, rows, cols, typ, xq, xd)
    oracle.kro_silu_mul(g.ctypes.data, u.ctypes.data, rows)
    assert np.array_equal(bits(hb.get(np.float32, rows)), bits(g))


@pytest.mark.parametrize("n,T", [(288, 37), (64, 5), (4096, 3)])
def test_rows_ops_match_single_calls(dev, n, T):
    """krh_<op>_rows over T rows with padded and zero row strides gives each
    row the single call's bits and leaves the gaps between rows alone (the
    op-table binding's batched replay of model/transformer.c:366-376)"""
    H = K.hip
    rng = np.random.default_rng(n + T)
    pad = 36

    def rows_pair(width, dtype=np.float32, fill=True):
        a = (rng.standard_normal(T * width) * 3).astype(np.float32) if fill else np.zeros(T * width, np.float32)
        if dtype is not np.float32:
            a = np.zeros(T * width, dtype)
        return dev.put(a), dev.put(a.copy()), a.nbytes

    F = 4
    ld = n + pad
    x = dev.put((rng.standard_normal(T * ld) * 2).astype(np.float32))
    x_host = x.get(np.float32, T * ld).copy()
    x_host[ld:ld + n] = 0.0                                   # a row under the quantizers' tiny threshold
    K.check(H.krh_copy_h2d(x.ptr, x_host.ctypes.data, x_host.nbytes), "copy")
    w = dev.put(rng.standard_normal(n).astype(np.float32))

    # rmsnorm: w shared by every row (stride 0)
    o1, o2, nb = rows_pair(ld, fill=False)
    H.krh_rmsnorm_rows(o1.ptr, ld, x.ptr, ld, w.ptr, 0, n, 1e-5, T)
    for r in range(T):
        H.krh_rmsnorm(o2.ptr + F * r * ld, x.ptr + F * r * ld, w.ptr, n, 1e-5)
    ok()
    assert np.array_equal(o1.get(np.uint32, T * ld), o2.get(np.uint32, T * ld))

    # add (bias with stride 0, and a row-strided operand), silu_mul, gelu_mul
    for name, single in (("add", H.krh_add), ("silu_mul", H.krh_silu_mul), ("gelu_mul", H.krh_gelu_mul)):
        for xs in (0, ld):
            y1, y2, _ = rows_pair(ld)
            getattr(H, "krh_%s_rows" % name)(y1.ptr, ld, x.ptr, xs, n, T)
            for r in range(T):
                single(y2.ptr + F * r * ld, x.ptr + F * r * xs, n)
            ok()
            assert np.array_equal(y1.get(np.uint32, T * ld), y2.get(np.uint32, T * ld)), (name, xs)

    # rope: q and k rows of heads, cos/sin rows of consecutive positions
    hd = 64 if n >= 64 else 16
    nh, nkv = max(1, n // hd), max(1, n // hd // 2)
    ldq, ldk, h2 = nh * hd + 8, nkv * hd + 4, hd // 2
    q1, q2, _ = rows_pair(ldq)
    k1, k2, _ = rows_pair(ldk)
    cs = dev.put(rng.uniform(-1, 1, (T + 3) * h2).astype(np.float32))
    sn = dev.put(rng.uniform(-1, 1, (T + 3) * h2).astype(np.float32))
    H.krh_rope_rows(q1.ptr, ldq, k1.ptr, ldk, cs.ptr + F * 3 * h2, h2, sn.ptr + F * 3 * h2, h2, hd, nh, nkv, T)
    for r in range(T):
        H.krh_rope(q2.ptr + F * r * ldq, k2.ptr + F * r * ldk, cs.ptr + F * (3 + r) * h2, sn.ptr + F * (3 + r) * h2,
                   hd, nh, nkv)
    ok()
    assert np.array_equal(q1.get(np.uint32, T * ldq), q2.get(np.uint32, T * ldq))
    assert np.array_equal(k1.get(np.uint32, T * ldk), k2.get(np.uint32, T * ldk))

    # quantize_row (one scale per row, scales 3 floats apart) and Q8_0 rows
    ldqb, ldd = n + 12, 3
    qa, qb = dev.zeros(T * ldqb), dev.zeros(T * ldqb)
    da, db = dev.zeros(F * T * ldd), dev.zeros(F * T * ldd)
    H.krh_quantize_row_rows(qa.ptr, ldqb, da.ptr, ldd, x.ptr, ld, n, T)
    for r in range(T):
        H.krh_quantize_row(qb.ptr + r * ldqb, db.ptr + F * r * ldd, x.ptr + F * r * ld, n)
    ok()
    assert np.array_equal(qa.get(np.int8, T * ldqb), qb.get(np.int8, T * ldqb))
    assert np.array_equal(da.get(np.uint32, T * ldd), db.get(np.uint32, T * ldd))
    ldd8 = n // 32 + 5
    qa, qb = dev.zeros(T * ldqb), dev.zeros(T * ldqb)
    da, db = dev.zeros(F * T * ldd8), dev.zeros(F * T * ldd8)
    H.krh_quantize_q8_rows(qa.ptr, ldqb, da.ptr, ldd8, x.ptr, ld, n, T)
    for r in range(T):
        H.krh_quantize_q8(qb.ptr + r * ldqb, db.ptr + F * r * ldd8, x.ptr + F * r * ld, n, 1)
    ok()
    assert np.array_equal(qa.get(np.int8, T * ldqb), qb.get(np.int8, T * ldqb))
    assert np.array_equal(da.get(np.uint32, T * ldd8), db.get(np.uint32, T * ldd8))


def test_rows_ops_reject_bad_shapes(dev):
    """misaligned Q8_0 rows and row counts past KRH_ROWS_MAX are refused
    before any launch, with ML_E_SHAPE"""
    H = K.hip
    buf = dev.zeros(4096)
    H.krh_quantize_q8_rows(buf.ptr, 32, buf.ptr + 1024, 1, buf.ptr + 2048 + 4, 32, 32, 2)
    assert H.krh_status() == K.ML_E_SHAPE
    H.krh_clear_error()
    H.krh_add_rows(buf.ptr, 0, buf.ptr, 0, 4, 65536)
    assert H.krh_status() == K.ML_E_SHAPE
    H.krh_clear_error()
    ok()


@pytest.mark.parametrize("rows,cols,typ,d16", [(768, 288, K.ML_Q8_0, 0), (4864, 896, K.ML_Q4_0, 1),
                                               (14336, 4096, K.ML_Q8_0, 1), (40, 96, K.ML_Q8_0, 0)])
def test_matvec_fused_op_sequences(dev, rows, cols, typ, d16):
    """The launches the op-table binding fuses the reference's per-op calls
    into, each with every effect of those calls: krh_matvec_swiglu_keep
    (h = silu(w1 x) * (w3 x) and u = w3 x), krh_matvec_residual (y = W x,
    r += y) and krh_matvec_multi (three products of one input), bit for bit
    against the oracle's matvec, silu_mul and add"""
    H = K.hip
    mats = [rand_mat(rows, cols, typ, d16) for _ in range(2)]
    W1, W3 = (dmat(dev, q, d, dh, rows, cols, typ, d16) for q, d, dh in mats)
    xq, xd = O.quantize(f32(RNG.normal(0, 1, cols) * 30))
    xqb, xdb = dev.put(xq), dev.put(xd)
    g = oracle_matvec(mats[0][0], mats[0][1], rows, cols, typ, xq, xd)
    u = oracle_matvec(mats[1][0], mats[1][1], rows, cols, typ, xq, xd)
    h = g.copy()
    oracle.kro_silu_mul(h.ctypes.data, u.ctypes.data, rows)

    hb, ub = dev.zeros(4 * rows), dev.zeros(4 * rows)
    H.krh_matvec_swiglu_keep(hb.ptr, ub.ptr, C.byref(W1), C.byref(W3), xqb.ptr, xdb.ptr)
    ok()
    assert np.array_equal(bits(hb.get(np.float32, rows)), bits(h))
    assert np.array_equal(bits(ub.get(np.float32, rows)), bits(u))

    r0 = f32(RNG.normal(0, 1, rows))
    rb, yb = dev.put(r0), dev.zeros(4 * rows)
    H.krh_matvec_residual(rb.ptr, yb.ptr, C.byref(W1), xqb.ptr, xdb.ptr)
    ok()
    assert np.array_equal(bits(yb.get(np.float32, rows)), bits(g))
    assert np.array_equal(bits(rb.get(np.float32, rows)), bits((r0 + g).astype(np.float32)))

    # three matrices of different row counts
    rws = [rows, max(2, rows // 4), max(2, rows // 4) + 2]
    ms = [rand_mat(r, cols, typ, d16) for r in rws]
    Ws = [dmat(dev, q, d, dh, r, cols, typ, d16) for (q, d, dh), r in zip(ms, rws)]
    ys = [dev.zeros(4 * r) for r in rws]
    yp = (C.c_void_p * 3)(*[y.ptr for y in ys])
    wp = (C.c_void_p * 3)(*[C.addressof(W) for W in Ws])
    for nmat in (3, 2):
        H.krh_matvec_multi(yp, wp, nmat, xqb.ptr, xdb.ptr)
        ok()
        for (q, d, dh), r, y in list(zip(ms, rws, ys))[:nmat]:
            assert np.array_equal(bits(y.get(np.float32, r)), bits(oracle_matvec(q, d, r, cols, typ, xq, xd)))


@pytest.mark.parametrize("dim,nh,nkv,hd,typ,vtyp,bias,hidden", [(288, 6, 6, 48, K.ML_Q8_0, K.ML_Q8_0, 0, 768),
                                                                 (896, 14, 2, 64, K.ML_Q4_0, K.ML_Q8_0, 1, 4864),
                                                                 (4096, 32, 8, 128, K.ML_Q8_0, K.ML_Q8_0, 0, 14336),
                                                                 (5120, 40, 8, 128, K.ML_Q8_0, K.ML_Q8_0, 0, 13824)])
def test_matvec_keep_prologues(dev, dim, nh, nkv, hd, typ, vtyp, bias, hidden):
    """the fused-norm and float-input launches that also store their
    prologue's results (the op-table binding's replacement of the reference's
    rmsnorm, quantize_q8 and products, model/transformer.c:270-293): xb, the
    Q8_0 of xb (or of x), and every product, bit for bit against the oracle's
    rmsnorm, quantize, matvec, add, rope and silu_mul. Inputs longer than the
    prologue keeps in registers (4864, 5120, 13824, 14336) take the prologue
    staged through LDS, which stores the same results."""
    H = K.hip
    qd, kvd, pos = nh * hd, nkv * hd, 17
    x = f32(RNG.normal(0, 2, dim))
    nw = f32(RNG.normal(1, 0.1, dim))
    xb_want = np.zeros(dim, np.float32)
    oracle.kro_rmsnorm(xb_want.ctypes.data, x.ctypes.data, nw.ctypes.data, dim, C.c_float(1e-5))
    xq_want, xd_want = O.quantize(xb_want)
    xdev, nwdev = dev.put(x), dev.put(nw)

    def kept(xbb, xqb, xdb, want_xb=True):
        if want_xb:
            assert np.array_equal(bits(xbb.get(np.float32, dim)), bits(xb_want))
        assert np.array_equal(xqb.get(np.int8, dim), xq_want)
        assert np.array_equal(bits(xdb.get(np.float32, dim // 32)), bits(xd_want))

    # q, k, v with the attention norm, biases and RoPE into the staging rows
    typs = (typ, typ, vtyp)
    mats = [rand_mat(r, dim, t, 1) for r, t in zip((qd, kvd, kvd), typs)]
    Ws = [dmat(dev, q, d, dh, r, dim, t, 1) for (q, d, dh), r, t in zip(mats, (qd, kvd, kvd), typs)]
    biases = [f32(RNG.normal(0, 0.02, r)) for r in (qd, kvd, kvd)]
    cs, sn = f32(RNG.uniform(-1, 1, 40 * hd // 2)), f32(RNG.uniform(-1, 1, 40 * hd // 2))
    qb, kb, vb = dev.zeros(4 * qd), dev.zeros(4 * kvd), dev.zeros(4 * kvd)
    xbb, xqb, xdb = dev.zeros(4 * dim), dev.zeros(dim), dev.zeros(4 * dim // 32)
    bb = [dev.put(b) if bias else None for b in biases]
    H.krh_rmsnorm_matvec_qkv_keep(qb.ptr, kb.ptr, vb.ptr, C.byref(Ws[0]), C.byref(Ws[1]), C.byref(Ws[2]),
                                  *[b.ptr if b else None for b in bb], xdev.ptr, nwdev.ptr, C.c_float(1e-5),
                                  dev.put(cs).ptr, dev.put(sn).ptr, hd, dev.put(np.array([pos], np.int32)).ptr,
                                  xbb.ptr, xqb.ptr, xdb.ptr)
    ok()
    kept(xbb, xqb, xdb)
    outs = []
    for (q, d, dh), r, b, t in zip(mats, (qd, kvd, kvd), biases, typs):
        y = oracle_matvec(q, d, r, dim, t, xq_want, xd_want)
        if bias:
            oracle.kro_add(y.ctypes.data, b.ctypes.data, r)
        outs.append(y)
    c0, s0 = f32(cs[pos * hd // 2:(pos + 1) * hd // 2]), f32(sn[pos * hd // 2:(pos + 1) * hd // 2])
    oracle.kro_rope(outs[0].ctypes.data, outs[1].ctypes.data, c0.ctypes.data, s0.ctypes.data, hd, nh, nkv)
    for got, want, r in ((qb, outs[0], qd), (kb, outs[1], kvd), (vb, outs[2], kvd)):
        assert np.array_equal(bits(got.get(np.float32, r)), bits(want))

    # w1, w3 with the FFN norm: h = silu(w1 xb) * (w3 xb), u = w3 xb
    m1, m3 = rand_mat(hidden, dim, typ, 1), rand_mat(hidden, dim, typ, 1)
    W1, W3 = dmat(dev, *m1, hidden, dim, typ, 1), dmat(dev, *m3, hidden, dim, typ, 1)
    hb, ub = dev.zeros(4 * hidden), dev.zeros(4 * hidden)
    xbb, xqb, xdb = dev.zeros(4 * dim), dev.zeros(dim), dev.zeros(4 * dim // 32)
    H.krh_rmsnorm_matvec_swiglu_keep(hb.ptr, ub.ptr, C.byref(W1), C.byref(W3), xdev.ptr, nwdev.ptr,
                                     C.c_float(1e-5), xbb.ptr, xqb.ptr, xdb.ptr)
    ok()
    kept(xbb, xqb, xdb)
    g = oracle_matvec(m1[0], m1[1], hidden, dim, typ, xq_want, xd_want)
    u = oracle_matvec(m3[0], m3[1], hidden, dim, typ, xq_want, xd_want)
    h = g.copy()
    oracle.kro_silu_mul(h.ctypes.data, u.ctypes.data, hidden)
    assert np.array_equal(bits(hb.get(np.float32, hidden)), bits(h))
    assert np.array_equal(bits(ub.get(np.float32, hidden)), bits(u))

    # w2 from the float h, quantized in the launch: y = W2 q8(h), r += y
    m2 = rand_mat(dim, hidden, vtyp, 1)
    W2 = dmat(dev, *m2, dim, hidden, vtyp, 1)
    r0 = f32(RNG.normal(0, 1, dim))
    rb, yb = dev.put(r0), dev.zeros(4 * dim)
    hq, hd_ = dev.zeros(hidden), dev.zeros(4 * hidden // 32)
    H.krh_matvec_f_residual_keep(rb.ptr, yb.ptr, C.byref(W2), dev.put(h).ptr, hq.ptr, hd_.ptr)
    ok()
    hq_want, hd_want = O.quantize(h)
    assert np.array_equal(hq.get(np.int8, hidden), hq_want)
    assert np.array_equal(bits(hd_.get(np.float32, hidden // 32)), bits(hd_want))
    y = oracle_matvec(m2[0], m2[1], dim, hidden, vtyp, hq_want, hd_want)
    assert np.array_equal(bits(yb.get(np.float32, dim)), bits(y))
    assert np.array_equal(bits(rb.get(np.float32, dim)), bits((r0 + y).astype(np.float32)))
