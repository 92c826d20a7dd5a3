"""Pins the oracle (oracle/kro*.c) before anything is checked against it:
against the reference's own scalar build compiled from its sources
(oracle/_ref), the reference's known-answer tests, the host C library, and
closed forms. CPU only."""
import ctypes as C
import os

import numpy as np
import pytest

import krafla as K
import oracle_lib as O
from oracle_lib import oracle, ref

needs_ref = pytest.mark.skipif(ref is None, reason="oracle/_ref not built (needs /root/reference at build time)")
RNG = np.random.default_rng(1234)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---- expf: the reference calls the C library's expf ----

def test_expf_exhaustive_vs_libm():
    # every float32 input; the restated algorithm must equal the host libm
    assert oracle.kro_expf_mismatches(0, 1 << 32, os.cpu_count() or 8) == 0


def test_expf_specials():
    for x, want in [(0.0, 1.0), (-np.inf, 0.0), (np.inf, np.inf), (89.0, np.inf), (-104.0, 0.0), (1.0, np.e)]:
        got = oracle.kro_expf(x)
        assert got == np.float32(want) or abs(got - want) <= 1e-6 * abs(want)
    assert np.isnan(oracle.kro_expf(float("nan")))


# ---- quantize_q8: known answers (tests/test_quant.c:28-70) and the rule ----

def test_quantize_ties_kat():
    x = np.zeros(32, dtype=np.float32)
    x[:6] = [127.0, 0.5, -0.5, 1.5, 2.5, -2.5]
    q, d = O.quantize(x)
    assert d[0] == 1.0
    assert q[1:6].tolist() == [1, -1, 2, 3, -3]


def test_quantize_clamp_zero_tiny_kat():
    x = f32(RNG.uniform(-1, 1, 96))
    x[3], x[9] = -5.0, 4.999
    x[32:64] = 0.0
    x[64:96] = [0.0 if i % 3 == 0 else (1e-37 if i % 3 == 1 else -2e-37) for i in range(32)]
    q, d = O.quantize(x)
    assert q[3] == -127 and q.min() >= -127 and q.max() <= 127
    assert d[1] == 0.0 and not q[32:64].any()
    assert d[2] == 0.0 and not q[64:96].any()


def test_quantize_roundtrip_bound():
    x = f32(RNG.uniform(-3, 3, 256))
    q, d = O.quantize(x)
    err = np.abs(x - q * np.repeat(d, 32))
    assert np.all(err <= np.repeat(d, 32) / 2 + 1e-7)


def test_quantize_closed_form():
    # numpy float32 arithmetic of the rule, element by element
    x = f32(RNG.normal(0, 2, 4096))
    q, d = O.quantize(x)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    id_ = (np.float32(127.0) / amax).astype(np.float32)
    v = np.trunc((xb * id_[:, None]).astype(np.float32) + np.copysign(np.float32(0.5), xb)).astype(np.float32)
    assert np.array_equal(np.clip(v, -127, 127).astype(np.int8).ravel(), q)
    assert np.array_equal(bits(amax / np.float32(127.0)), bits(d))


@needs_ref
@pytest.mark.parametrize("k", [32, 4096])
def test_quantize_matches_reference(k):
    for scale in [1e-3, 1.0, 1e3]:
        x = f32(RNG.normal(0, scale, k))
        x[:32] = 0.0 if k > 32 else x[:32]
        q0, d0 = O.quantize(x)
        q1 = np.zeros(k, dtype=np.int8)
        d1 = np.zeros(k // 32, dtype=np.float32)
        a = O.qact(q1, d1)
        ref.ml_k_quantize_q8_scalar(C.byref(a), x.ctypes.data, k)
        assert np.array_equal(q0, q1) and np.array_equal(bits(d0), bits(d1))


# ---- matvec: exact int dots (closed form) and the reference's float order ----

def rand_mat(rows, cols, typ, rng=RNG):
    if typ == K.ML_Q8_0:
        q = rng.integers(-127, 128, rows * cols).astype(np.int8)
    else:
        q = rng.integers(0, 256, rows * cols // 2).astype(np.uint8)
    d = f32(np.abs(rng.normal(0, 0.01, rows * cols // 32)))
    return q, d


def rand_act(k, rng=RNG):
    return O.quantize(f32(rng.normal(0, 1, k)))


def int_dots(q, typ, rows, cols, xq):
    nb = cols // 32
    if typ == K.ML_Q8_0:
        w = q.astype(np.int64).reshape(rows, nb, 32)
    else:
        p = q.reshape(rows, nb, 16)
        w = np.concatenate([(p & 15).astype(np.int64) - 8, (p >> 4).astype(np.int64) - 8], axis=2)
    return (w * xq.astype(np.int64).reshape(1, nb, 32)).sum(axis=2)


@pytest.mark.parametrize("typ", [K.ML_Q8_0, K.ML_Q4_0])
def test_block_dots_brute_force(typ):
    rows, cols = 7, 256
    q, d = rand_mat(rows, cols, typ)
    xq, xd = rand_act(cols)
    W = O.qtensor(q, d, rows, cols, typ)
    s = np.zeros(rows * cols // 32, dtype=np.int32)
    oracle.kro_block_dots(s.ctypes.data, C.byref(W), C.byref(O.qact(xq, xd)), 0, rows)
    assert np.array_equal(s.reshape(rows, -1), int_dots(q, typ, rows, cols, xq))


@pytest.mark.parametrize("typ", [K.ML_Q8_0, K.ML_Q4_0])
def test_matvec_unit_scales_exact(typ):
    # with unit scales the result is the exact integer sum (tests/test_kernels.c:103)
    rows, cols = 5, 96
    q, _ = rand_mat(rows, cols, typ)
    d = np.ones(rows * cols // 32, dtype=np.float32)
    xq, _ = rand_act(cols)
    xd = np.ones(cols // 32, dtype=np.float32)
    W = O.qtensor(q, d, rows, cols, typ)
    y = np.zeros(rows, dtype=np.float32)
    fn = oracle.kro_matvec_q8 if typ == K.ML_Q8_0 else oracle.kro_matvec_q4
    fn(y.ctypes.data, C.byref(W), C.byref(O.qact(xq, xd)), 0, rows)
    assert np.array_equal(y, int_dots(q, typ, rows, cols, xq).sum(axis=1).astype(np.float32))


def test_matvec_order_closed_form():
    # sum += ((float)s * wd) * xd in block order, evaluated in numpy float32
    rows, cols = 3, 8288
    q, d = rand_mat(rows, cols, K.ML_Q8_0)
    xq, xd = rand_act(cols)
    W = O.qtensor(q, d, rows, cols, K.ML_Q8_0)
    y = np.zeros(rows, dtype=np.float32)
    oracle.kro_matvec_q8(y.ctypes.data, C.byref(W), C.byref(O.qact(xq, xd)), 0, rows)
    s = int_dots(q, K.ML_Q8_0, rows, cols, xq).astype(np.float32)
    t = (s * d.reshape(rows, -1)).astype(np.float32) * xd[None, :]
    want = np.zeros(rows, dtype=np.float32)
    for b in range(cols // 32):
        want = (want + t[:, b]).astype(np.float32)
    assert np.array_equal(bits(y), bits(want))
    # a transposed or reordered sum would differ: check the test can tell
    assert not np.array_equal(bits(t.sum(axis=1, dtype=np.float32)), bits(want)) or rows == 0


@needs_ref
@pytest.mark.parametrize("typ", [K.ML_Q8_0, K.ML_Q4_0])
@pytest.mark.parametrize("rows,cols", [(1, 32), (3, 96), (64, 256), (7, 8288), (17, 4096)])
def test_matvec_matches_reference(typ, rows, cols):
    q, d = rand_mat(rows, cols, typ)
    xq, xd = rand_act(cols)
    W = O.qtensor(q, d, rows, cols, typ)
    x = O.qact(xq, xd)
    y0 = np.full(rows + 2, 12345.0, dtype=np.float32)
    y1 = y0.copy()
    name = "matvec_q8" if typ == K.ML_Q8_0 else "matvec_q4"
    getattr(oracle, "kro_" + name)(y0.ctypes.data, C.byref(W), C.byref(x), 1, rows)
    getattr(ref, "ml_k_%s_scalar" % name)(y1.ctypes.data, C.byref(W), C.byref(x), 1, rows)
    assert np.array_equal(bits(y0), bits(y1))
    assert y0[0] == 12345.0 and y0[rows] == 12345.0  # rows outside [r0, r1) untouched


# ---- float kernels vs the reference's scalar kernels ----

@needs_ref
@pytest.mark.parametrize("n", [32, 288, 4096])
def test_rmsnorm_softmax_silu_add_match_reference(n):
    x, w, u = f32(RNG.normal(0, 1, n)), f32(RNG.normal(1, 0.1, n)), f32(RNG.normal(0, 1, n))
    for fn_o, fn_r, args in [
        ("kro_rmsnorm", "ml_k_rmsnorm_scalar", lambda o: (o.ctypes.data, x.ctypes.data, w.ctypes.data, n, 1e-5)),
    ]:
        o0, o1 = np.zeros(n, np.float32), np.zeros(n, np.float32)
        getattr(oracle, fn_o)(*args(o0))
        getattr(ref, fn_r)(*args(o1))
        assert np.array_equal(bits(o0), bits(o1))
    s0, s1 = f32(RNG.normal(0, 3, n)), None
    s1 = s0.copy()
    oracle.kro_softmax(s0.ctypes.data, n)
    ref.ml_k_softmax_scalar(s1.ctypes.data, n)
    assert np.array_equal(bits(s0), bits(s1))
    g0 = f32(RNG.normal(0, 4, n))
    g1 = g0.copy()
    oracle.kro_silu_mul(g0.ctypes.data, u.ctypes.data, n)
    ref.ml_k_silu_mul_scalar(g1.ctypes.data, u.ctypes.data, n)
    assert np.array_equal(bits(g0), bits(g1))
    a0 = x.copy()
    a1 = x.copy()
    oracle.kro_add(a0.ctypes.data, u.ctypes.data, n)
    ref.ml_k_add_scalar(a1.ctypes.data, u.ctypes.data, n)
    assert np.array_equal(bits(a0), bits(a1))


@needs_ref
def test_rope_dot_axpy_match_reference():
    hd, nh, nkv = 64, 4, 2
    q0, k0 = f32(RNG.normal(0, 1, hd * nh)), f32(RNG.normal(0, 1, hd * nkv))
    cs, sn = f32(RNG.uniform(-1, 1, hd // 2)), f32(RNG.uniform(-1, 1, hd // 2))
    q1, k1 = q0.copy(), k0.copy()
    oracle.kro_rope(q0.ctypes.data, k0.ctypes.data, cs.ctypes.data, sn.ctypes.data, hd, nh, nkv)
    ref.ml_k_rope_scalar(q1.ctypes.data, k1.ctypes.data, cs.ctypes.data, sn.ctypes.data, hd, nh, nkv)
    assert np.array_equal(bits(q0), bits(q1)) and np.array_equal(bits(k0), bits(k1))
    rows, ld = 37, 96
    kk = f32(RNG.normal(0, 1, rows * ld))
    s0, s1 = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
    oracle.kro_dot_f32(s0.ctypes.data, q1.ctypes.data, kk.ctypes.data, ld, rows, hd, 0.125)
    ref.ml_k_dot_f32_scalar(s1.ctypes.data, q1.ctypes.data, kk.ctypes.data, ld, rows, hd, 0.125)
    assert np.array_equal(bits(s0), bits(s1))
    y0 = f32(RNG.normal(0, 1, hd))
    y1 = y0.copy()
    oracle.kro_axpy_f32(y0.ctypes.data, s0.ctypes.data, kk.ctypes.data, ld, rows, hd)
    ref.ml_k_axpy_f32_scalar(y1.ctypes.data, s0.ctypes.data, kk.ctypes.data, ld, rows, hd)
    assert np.array_equal(bits(y0), bits(y1))


@needs_ref
@pytest.mark.parametrize("typ", [K.ML_Q8_0, K.ML_Q4_0])
def test_dequant_and_q4_rule_match_reference(typ):
    q, d = rand_mat(4, 128, typ)
    W = O.qtensor(q, d, 4, 128, typ)
    o0, o1 = np.zeros(128, np.float32), np.zeros(128, np.float32)
    oracle.kro_dequant_row(o0.ctypes.data, C.byref(W), 2)
    ref.ml_dequant_row(o1.ctypes.data, C.byref(W), 2)
    assert np.array_equal(bits(o0), bits(o1))
    x = f32(RNG.normal(0, 1, 128))
    x[32:64] = 0
    qa, da = np.zeros(64, np.uint8), np.zeros(4, np.float32)
    qb, db = qa.copy(), da.copy()
    oracle.kro_quantize_row_q4(qa.ctypes.data, da.ctypes.data, x.ctypes.data, 128)
    ref.ml_quantize_row_q4(qb.ctypes.data, db.ctypes.data, x.ctypes.data, 128)
    assert np.array_equal(qa, qb) and np.array_equal(bits(da), bits(db))


def test_argmax_ties_lowest():
    # tests/test_sampler.c:33-40
    v = np.zeros(64, np.float32)
    v[40] = v[9] = 3.0
    assert oracle.kro_argmax(v.ctypes.data, 64) == 9
    v = np.full(8, -np.inf, np.float32)
    assert oracle.kro_argmax(v.ctypes.data, 8) == 0


def test_f16_widening_closed_form():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.kro_f16_to_f32(int(v)) for v in h[::97]], dtype=np.float32)
    w = want[::97]
    finite = np.isfinite(w)
    assert np.array_equal(bits(got[finite]), bits(w[finite]))


# ---- F16 and Q8 KV caches (k_scalar.c:124-155, ops/ops.c:81-96) ----

def test_tanhf_exhaustive_vs_libm():
    """the restated tanhf and expm1f equal the host C library's (glibc 2.35,
    which the reference calls) on every float32 input"""
    assert O.oracle.kro_tanhf_mismatches(0, 1 << 32, os.cpu_count() or 8) == 0


def test_tanhf_specials():
    for x, want in [(0.0, 0.0), (-0.0, -0.0), (float("inf"), 1.0), (float("-inf"), -1.0), (30.0, 1.0)]:
        got = O.oracle.kro_tanhf(x)
        assert got == want and np.signbit(np.float32(got)) == np.signbit(np.float32(want))
    assert np.isnan(O.oracle.kro_tanhf(float("nan")))


@needs_ref
@pytest.mark.parametrize("n", [1, 77, 4096])
def test_gelu_softcap_match_reference(n):
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    g[: min(n, 4)] = [0.0, -0.0, 1e-30, -40.0][: min(n, 4)]
    u = rng.standard_normal(n).astype(np.float32)
    a, b = g.copy(), g.copy()
    O.oracle.kro_gelu_mul(a.ctypes.data, u.ctypes.data, n)
    ref.ml_k_gelu_mul_scalar(b.ctypes.data, u.ctypes.data, n)
    assert np.array_equal(bits(a), bits(b))
    x = (rng.standard_normal(3 * n) * 30).astype(np.float32)
    a, b = x.copy(), x.copy()
    O.oracle.kro_softcap_rows(a.ctypes.data, n, 3, n - (n > 1), 7.5)
    ref.ml_softcap_rows(b.ctypes.data, n, 3, n - (n > 1), 7.5)
    assert np.array_equal(bits(a), bits(b))


def test_f32_to_f16_exhaustive_vs_ieee():
    # every float32 input against the x86 F16C conversion (IEEE round to
    # nearest even); NaN inputs become the quiet NaN 0x7e00 with their sign
    bad = oracle.kro_f32_to_f16_mismatches(0, 1 << 32, os.cpu_count() or 8)
    if bad == 2**64 - 1:
        pytest.skip("host CPU without F16C")
    assert bad == 0


def test_f32_to_f16_sample_vs_numpy():
    # the same rule against numpy's IEEE cast on a sample of every binade
    u = np.concatenate([RNG.integers(0, 1 << 32, 1 << 20, dtype=np.uint64),
                        np.arange(0x477FE000, 0x47800100, dtype=np.uint64),
                        np.arange(0x33000000 - 256, 0x33000000 + 256, dtype=np.uint64),
                        np.arange(0x387FFF00, 0x38800100, dtype=np.uint64)]).astype(np.uint32)
    u = np.concatenate([u, u | np.uint32(0x80000000)])
    out = np.empty(1, np.uint16)
    got = np.empty(len(u), np.uint16)
    for i, b in enumerate(u[:4096]):
        oracle.kro_f32_to_f16_range(out.ctypes.data, int(b), 1)
        got[i] = out[0]
    x = u[:4096].view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    want = np.where(np.isnan(x), ((u[:4096] >> 16) & 0x8000).astype(np.uint16) | np.uint16(0x7E00), want)
    assert np.array_equal(got[:4096], want)


@needs_ref
def test_f32_to_f16_matches_reference():
    x = np.concatenate([f32(RNG.normal(0, 1, 4000)), f32(RNG.normal(0, 3e4, 1000)), f32(RNG.uniform(-1e-4, 1e-4, 1000)),
                        f32([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8,
                             np.inf, -np.inf, np.nan])])
    got = [oracle.kro_f32_to_f16(float(v)) for v in x]
    want = [ref.ml_f32_to_f16(float(v)) for v in x]
    assert got == want


def q8_rows(n):
    return RNG.integers(-127, 128, n).astype(np.int8)


@needs_ref
@pytest.mark.parametrize("n", [1, 7, 32, 64, 128, 300])
@pytest.mark.parametrize("rows", [1, 3, 4, 5, 9])
def test_kv_kernels_match_reference(n, rows):
    # the shapes of tests/test_kernels.c:334-426 (strided rows and scales)
    A = f32(RNG.uniform(0, 1, n))
    K16 = np.array([oracle.kro_f32_to_f16(float(v)) for v in RNG.uniform(0, 1, (n + 3) * rows)], np.uint16)
    a = f32(RNG.uniform(0, 1, rows))
    s0, s1 = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
    oracle.kro_dot_f16(s0.ctypes.data, A.ctypes.data, K16.ctypes.data, n + 3, rows, n, 0.125)
    ref.ml_k_dot_f16_scalar(s1.ctypes.data, A.ctypes.data, K16.ctypes.data, n + 3, rows, n, 0.125)
    assert np.array_equal(bits(s0), bits(s1))
    y0 = f32(RNG.uniform(-2, 2, n))
    y1 = y0.copy()
    oracle.kro_axpy_f16(y0.ctypes.data, a.ctypes.data, K16.ctypes.data, n + 3, rows, n)
    ref.ml_k_axpy_f16_scalar(y1.ctypes.data, a.ctypes.data, K16.ctypes.data, n + 3, rows, n)
    assert np.array_equal(bits(y0), bits(y1))
    Kq, q, dk = q8_rows((n + 5) * rows), q8_rows(n), f32(RNG.uniform(0.001, 0.05, 3 * rows))
    oracle.kro_dot_q8(s0.ctypes.data, q.ctypes.data, 0.02, Kq.ctypes.data, dk.ctypes.data, n + 5, 3, rows, n, 0.125)
    ref.ml_k_dot_q8_scalar(s1.ctypes.data, q.ctypes.data, 0.02, Kq.ctypes.data, dk.ctypes.data, n + 5, 3, rows, n,
                           0.125)
    assert np.array_equal(bits(s0), bits(s1))
    dx = f32(RNG.uniform(0.001, 0.05, 2 * rows))
    y0 = f32(RNG.uniform(-2, 2, n))
    y1 = y0.copy()
    oracle.kro_axpy_q8(y0.ctypes.data, a.ctypes.data, Kq.ctypes.data, dx.ctypes.data, n + 5, 2, rows, n)
    ref.ml_k_axpy_q8_scalar(y1.ctypes.data, a.ctypes.data, Kq.ctypes.data, dx.ctypes.data, n + 5, 2, rows, n)
    assert np.array_equal(bits(y0), bits(y1))


def test_dot_q8_exact_integer_sum():
    # unit scales: the score is the int32 dot itself, exactly (|sum| < 2^24)
    n, rows = 128, 9
    K8, q = q8_rows(n * rows), q8_rows(n)
    dk = np.ones(rows, np.float32)
    s = np.zeros(rows, np.float32)
    oracle.kro_dot_q8(s.ctypes.data, q.ctypes.data, 1.0, K8.ctypes.data, dk.ctypes.data, n, 1, rows, n, 1.0)
    want = (K8.reshape(rows, n).astype(np.int64) * q.astype(np.int64)).sum(axis=1)
    assert np.array_equal(s.astype(np.int64), want)
    # the float factors apply in the order ((float)sum * (dq * scale)) * dk
    dk = f32(RNG.uniform(0.001, 0.05, rows))
    oracle.kro_dot_q8(s.ctypes.data, q.ctypes.data, 0.02, K8.ctypes.data, dk.ctypes.data, n, 1, rows, n, 0.125)
    c = np.float32(0.02) * np.float32(0.125)
    assert np.allclose(s, want * float(c) * dk, rtol=1e-6)


def test_axpy_q8_weight_then_value():
    # y += (a_t * dx_t) * x_t: with x = 1 the increments are the weights a_t * dx_t
    n, rows = 16, 5
    a, dx = f32(RNG.uniform(0, 1, rows)), f32(RNG.uniform(0.001, 0.05, rows))
    X = np.ones(n * rows, np.int8)
    y = np.zeros(n, np.float32)
    oracle.kro_axpy_q8(y.ctypes.data, a.ctypes.data, X.ctypes.data, dx.ctypes.data, n, 1, rows, n)
    want = np.float32(0.0)
    for t in range(rows):
        want = np.float32(want + np.float32(a[t] * dx[t]))
    assert np.all(bits(y) == bits(np.full(n, want, np.float32)))


@needs_ref
@pytest.mark.parametrize("n", [32, 64, 128, 300])
def test_quantize_row_matches_reference(n):
    for x in (f32(RNG.normal(0, 2, n)), np.zeros(n, np.float32), f32(np.full(n, 1e-37)),
              f32(np.r_[[127.0, 0.5, -0.5, 1.5, 2.5, -2.5], np.zeros(n - 6)])):
        q0, q1 = np.zeros(n, np.int8), np.zeros(n, np.int8)
        d0, d1 = np.zeros(1, np.float32), np.zeros(1, np.float32)
        oracle.kro_quantize_row(q0.ctypes.data, d0.ctypes.data, x.ctypes.data, n)
        ref.ml_quantize_row(q1.ctypes.data, d1.ctypes.data, x.ctypes.data, n)
        assert np.array_equal(q0, q1) and bits(d0)[0] == bits(d1)[0]


def test_quantize_row_one_scale():
    # one scale for the whole row, the largest magnitude at +-127, ties away from zero
    x = f32(np.r_[[127.0, 0.5, -0.5, 1.5, 2.5, -2.5], RNG.uniform(-1, 1, 122)])
    q, d = np.zeros(128, np.int8), np.zeros(1, np.float32)
    oracle.kro_quantize_row(q.ctypes.data, d.ctypes.data, x.ctypes.data, 128)
    assert d[0] == 1.0 and q[0] == 127 and q[1:6].tolist() == [1, -1, 2, 3, -3]


# ---- whole model: the oracle's forward vs the reference's ml_run ----

SMALL = {
    "c1_q8": dict(K.CONFIGS["stories15m_q8"]),
    "c1_q8_std01": dict(K.CONFIGS["stories15m_q8"], std=0.1, seed=11),
    "qwen_like_q4mix": dict(K.CONFIGS["qwen05b_mixed"], dim=128, n_layers=3, n_heads=4, n_kv_heads=2,
                            hidden_dim=256, vocab=512, max_seq=96, std=0.1),
    "llama3_rope_gqa_q4": dict(K.CONFIGS["llama1b_mixed"], dim=256, n_layers=2, n_heads=8, n_kv_heads=2,
                               hidden_dim=512, vocab=1000, max_seq=200, std=0.1, rope_orig_max_seq=64),
    "q8_f16_untied": dict(K.CONFIGS["llama8b_q8"], dim=256, n_layers=2, n_heads=4, n_kv_heads=1, hidden_dim=384,
                          vocab=700, max_seq=160, std=0.1),
    # the families' norms: q/k RMSNorm per head (Qwen3), post-norms (Gemma 3)
    "qk_norm_bias_gqa": dict(K.CONFIGS["qwen05b_mixed"], dim=128, n_layers=2, n_heads=4, n_kv_heads=2,
                             hidden_dim=256, vocab=512, max_seq=96, std=0.1, qk_norm=1),
    "post_norms_q8": dict(K.CONFIGS["stories15m_q8"], std=0.1, seed=3, post_norms=1),
    "qk_post_norms_f16": dict(K.CONFIGS["llama8b_q8"], dim=256, n_layers=2, n_heads=2, n_kv_heads=1,
                              hidden_dim=384, vocab=600, max_seq=128, std=0.1, qk_norm=1, post_norms=1),
    # attention windows and RoPE variants (ops/ops.c:127-128, model/transformer.c:16-38, :182-186)
    "window_all_layers": dict(K.CONFIGS["stories15m_q8"], std=0.1, seed=21, sliding_window=5),
    "window_local_rope_layers": dict(K.CONFIGS["qwen05b_mixed"], dim=128, n_layers=3, n_heads=4, n_kv_heads=2,
                                     hidden_dim=256, vocab=512, max_seq=96, std=0.1, rope_theta=1e6,
                                     sliding_window=4, layer_sliding=0b101, layer_local=0b001,
                                     rope_local_theta=1e4),
    "rope_linear": dict(K.CONFIGS["stories15m_q8"], std=0.1, seed=22, rope_type=K.ML_ROPE_LINEAR, rope_factor=4.0),
    "rope_yarn": dict(K.CONFIGS["stories15m_q8"], std=0.1, seed=23, rope_type=K.ML_ROPE_YARN, rope_factor=4.0,
                      rope_low_freq_factor=32.0, rope_high_freq_factor=1.0, rope_orig_max_seq=64,
                      rope_attn_factor=1.2),
    # GELU and soft-capping (k_scalar.c:100-105, ops/ops.c:98-101, :141, model/transformer.c:304)
    "gelu_softcap_gemma2": dict(K.CONFIGS["stories15m_q8"], std=0.1, seed=24, act=K.ML_ACT_GELU_TANH,
                                embed_scale=16.0, attn_softcap=5.0, final_softcap=3.0, sliding_window=6,
                                layer_sliding=0b101010),
    "gelu_post_qk_gemma3": dict(K.CONFIGS["qwen05b_mixed"], dim=128, n_layers=2, n_heads=4, n_kv_heads=2,
                                hidden_dim=256, vocab=512, max_seq=96, std=0.1, act=K.ML_ACT_GELU_TANH,
                                post_norms=1, qk_norm=1, final_softcap=8.0, rope_local_theta=1e4,
                                layer_local=0b01, layer_sliding=0b01, sliding_window=5),
}


@needs_ref
@pytest.mark.parametrize("name", sorted(SMALL))
def test_forward_matches_reference(name, workdir):
    path = os.path.join(workdir, name + ".mlb")
    K.gen_mlb(path, **SMALL[name])
    om = O.OracleModel(path)
    V = om.cfg.vocab
    toks = [int(t) for t in np.random.default_rng(5).integers(1, V, 12)]
    dump = path + ".logits"
    O.ref_ml_run(path, toks, len(toks), dump=dump)
    want = np.fromfile(dump, dtype=np.float32).reshape(len(toks), V)
    got = om.prefill(toks, 0, logits=True)
    assert np.array_equal(bits(got), bits(want))
    om.close()
    om = O.OracleModel(path)
    steps = min(om.cfg.max_seq, 60)
    ids_ref, _ = O.ref_ml_run(path, toks[:5], steps)
    assert np.array_equal(om.generate(toks[:5], steps), ids_ref)
    om.close()


LONG = {
    # the decode and batched attention at the context lengths of the 1B
    # workload (4,000-token prompt), on a one-layer model so the reference's
    # scalar loop runs it in seconds; llama3 RoPE scaling from position 64
    "long_gqa_q4mix": dict(K.CONFIGS["llama1b_mixed"], dim=64, n_layers=1, n_heads=4, n_kv_heads=2,
                           hidden_dim=128, vocab=256, max_seq=4200, std=0.1, rope_orig_max_seq=64),
    # one KV head for all query heads, a Q8 model with f16 scales
    "long_mqa_q8": dict(K.CONFIGS["llama8b_q8"], dim=64, n_layers=1, n_heads=2, n_kv_heads=1,
                        hidden_dim=96, vocab=200, max_seq=2200, std=0.1),
}


@needs_ref
@pytest.mark.parametrize("name", sorted(LONG))
def test_long_context_matches_reference(name, workdir):
    """every prefill row's logits over a prompt of max_seq - 200 tokens, and
    the ids of 100 decode steps after it (the per-token attention at those
    positions, ops/ops.c:124-180), equal the reference's ml_run"""
    path = os.path.join(workdir, name + ".mlb")
    K.gen_mlb(path, **LONG[name])
    om = O.OracleModel(path)
    V, P = om.cfg.vocab, om.cfg.max_seq - 200
    toks = [int(t) for t in np.random.default_rng(17).integers(1, V, P)]
    dump = path + ".logits"
    O.ref_ml_run(path, toks, len(toks), dump=dump)
    want = np.fromfile(dump, dtype=np.float32).reshape(len(toks), V)
    got = om.prefill(toks, 0, logits=True)
    assert np.array_equal(bits(got), bits(want))
    om.close()
    om = O.OracleModel(path)
    ids_ref, _ = O.ref_ml_run(path, toks, P + 100)
    assert np.array_equal(om.generate(toks, P + 100), ids_ref)
    om.close()


def test_hip_ml_run_guard_without_gpu(workdir):
    """the ISA=hip build keeps the reference's guard contract
    (app/main_guard.c:8-15): without a gfx950 device it exits 3"""
    exe = os.path.join(O.REF_DIR, "hip", "ml_run")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref/hip not built")
    if K.hip.krh_init() == K.ML_OK:
        pytest.skip("a gfx950 device is present")
    import subprocess
    path = os.path.join(workdir, "guard.mlb")
    K.gen_mlb(path, **dict(K.CONFIGS["stories15m_q8"], n_layers=1, vocab=64, max_seq=16))
    r = subprocess.run([exe, path, "--tokens", "1,2", "-n", "3"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 3 and "ISA=hip" in r.stderr


def test_binding_declares_every_export():
    """every C entry point of both libraries is declared with its argument
    types in the ctypes binding (an undeclared call would truncate pointers)"""
    import subprocess
    for lib, libpath in ((K.hip, K.LIB_HIP), (K.host, K.LIB_HOST)):
        out = subprocess.run(["nm", "-D", "--defined-only", libpath], capture_output=True, text=True).stdout
        syms = {l.split()[-1] for l in out.splitlines() if " T " in l}
        exported = {s for s in syms if s.startswith("krh_") or s.startswith("kr_")}
        assert exported and exported <= lib.declared(), sorted(exported - lib.declared())


def test_libraries_export_every_declared_function():
    """every function include/krafla_hip.h and include/krafla.h declare is
    exported by libkrafla_hip.so or libkrafla.so"""
    import re
    import subprocess
    exported = set()
    for libpath in (K.LIB_HIP, K.LIB_HOST):
        out = subprocess.run(["nm", "-D", "--defined-only", libpath], capture_output=True, text=True).stdout
        exported |= {l.split()[-1] for l in out.splitlines() if " T " in l}
    declared = set()
    for h in ("krafla_hip.h", "krafla.h"):
        text = open(os.path.join(O.ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        declared |= set(re.findall(r"^[A-Za-z_][\w \t\*]*?\b(krh?_\w+)\s*\(", text, flags=re.M))
    assert len(declared) > 50 and "krh_sample" in declared
    assert declared <= exported, sorted(declared - exported)


@needs_ref
@pytest.mark.parametrize("kv", ["q8", "f16"])
@pytest.mark.parametrize("name", ["c1_q8", "llama3_rope_gqa_q4", "qwen_like_q4mix"])
def test_forward_matches_reference_kv(name, kv, workdir):
    # ml_run --kv q8 / --kv f16 (app/ml_run.c:277-281): logits and greedy ids
    path = os.path.join(workdir, name + ".mlb")
    K.gen_mlb(path, **SMALL[name])
    kvt = K.ML_Q8_0 if kv == "q8" else K.ML_F16
    om = O.OracleModel(path, kvt)
    V = om.cfg.vocab
    toks = [int(t) for t in np.random.default_rng(6).integers(1, V, 12)]
    dump = path + "." + kv + ".logits"
    O.ref_ml_run(path, toks, len(toks), dump=dump, extra=("--kv", kv))
    want = np.fromfile(dump, dtype=np.float32).reshape(len(toks), V)
    got = om.prefill(toks, 0, logits=True)
    assert np.array_equal(bits(got), bits(want))
    om.close()
    om = O.OracleModel(path, kvt)
    steps = min(om.cfg.max_seq, 60)
    ids_ref, _ = O.ref_ml_run(path, toks[:5], steps, extra=("--kv", kv))
    assert np.array_equal(om.generate(toks[:5], steps), ids_ref)
    om.close()


def test_integration_stub_compiles(tmp_path):
    """the reference-side C stub in INTEGRATION.md compiles against include/
    and links against both libraries (no calls: no GPU here)"""
    import re
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    text = open(os.path.join(root, "INTEGRATION.md")).read()
    blocks = re.findall(r"```c\n(.*?)```", text, re.S)
    stub = next(b for b in blocks if "ml_main_hip" in b)
    src = tmp_path / "ml_run_hip.c"
    src.write_text(stub + "\nint main(void) { return 0; }\n")
    lib = os.path.join(root, "isa-lm_amd")
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", str(src), "-I", os.path.join(root, "include"),
                        "-L", lib, "-lkrafla", "-lkrafla_hip", "-Wl,-rpath," + lib, "-o", str(tmp_path / "stub")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
