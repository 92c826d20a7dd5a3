"""The families' layer path on the device: q/k RMSNorm per head (Qwen3) and
post-norms (Gemma 3), model/transformer.c:240-248. The heads' norm and RoPE
kernel against the oracle's kernels; whole-model logits and greedy ids
against the reference's ml_run, with each KV cache type."""
import ctypes as C
import os

import numpy as np
import pytest

import krafla as K
import oracle_lib as O
from oracle_lib import oracle

pytestmark = pytest.mark.gpu

FAMILY = {
    "qk_norm_bias_gqa": dict(K.CONFIGS["qwen05b_mixed"], dim=128, n_layers=2, n_heads=4, n_kv_heads=2,
                             hidden_dim=256, vocab=512, max_seq=96, std=0.1, qk_norm=1),
    "post_norms_q8": dict(K.CONFIGS["stories15m_q8"], std=0.1, seed=3, post_norms=1),
    "qk_post_norms_f16": dict(K.CONFIGS["llama8b_q8"], dim=256, n_layers=2, n_heads=2, n_kv_heads=1,
                              hidden_dim=384, vocab=600, max_seq=128, std=0.1, qk_norm=1, post_norms=1),
}
# attention windows and RoPE variants (ops/ops.c:127-128, model/transformer.c:16-38, :182-186)
VARIANTS = {
    "window_all_layers": dict(K.CONFIGS["stories15m_q8"], std=0.1, seed=21, sliding_window=5),
    "window_local_rope_layers": dict(K.CONFIGS["qwen05b_mixed"], dim=128, n_layers=3, n_heads=4, n_kv_heads=2,
                                     hidden_dim=256, vocab=512, max_seq=96, std=0.1, rope_theta=1e6,
                                     sliding_window=4, layer_sliding=0b101, layer_local=0b001,
                                     rope_local_theta=1e4),
    "rope_linear": dict(K.CONFIGS["stories15m_q8"], std=0.1, seed=22, rope_type=K.ML_ROPE_LINEAR, rope_factor=4.0),
    "rope_yarn": dict(K.CONFIGS["stories15m_q8"], std=0.1, seed=23, rope_type=K.ML_ROPE_YARN, rope_factor=4.0,
                      rope_low_freq_factor=32.0, rope_high_freq_factor=1.0, rope_orig_max_seq=64,
                      rope_attn_factor=1.2),
    "window_qk_norm": dict(K.CONFIGS["qwen05b_mixed"], dim=128, n_layers=2, n_heads=4, n_kv_heads=2,
                           hidden_dim=256, vocab=512, max_seq=96, std=0.1, qk_norm=1, sliding_window=6,
                           layer_sliding=0b10, layer_local=0b10, rope_local_theta=1e4),
}
# GELU and soft-capping (Gemma 2 / 3 shapes)
VARIANTS["gelu_softcap_gemma2"] = dict(K.CONFIGS["stories15m_q8"], std=0.1, seed=24, act=K.ML_ACT_GELU_TANH,
                                       embed_scale=16.0, attn_softcap=5.0, final_softcap=3.0, sliding_window=6,
                                       layer_sliding=0b101010)
VARIANTS["gelu_post_qk_gemma3"] = dict(K.CONFIGS["qwen05b_mixed"], dim=128, n_layers=2, n_heads=4, n_kv_heads=2,
                                       hidden_dim=256, vocab=512, max_seq=96, std=0.1, act=K.ML_ACT_GELU_TANH,
                                       post_norms=1, qk_norm=1, final_softcap=8.0, rope_local_theta=1e4,
                                       layer_local=0b01, layer_sliding=0b01, sliding_window=5)
# Gemma 2's 256-wide heads (two query heads sharing one KV head): the score
# tiles of such heads take the kernels' narrower position tiles
VARIANTS["gemma2_wide_heads"] = dict(K.CONFIGS["qwen05b_mixed"], dim=512, n_layers=2, n_heads=2, n_kv_heads=1,
                                     hidden_dim=1024, vocab=512, max_seq=96, std=0.1, act=K.ML_ACT_GELU_TANH,
                                     embed_scale=22.6, attn_softcap=50.0, final_softcap=30.0, sliding_window=6,
                                     layer_sliding=0b01, qkv_bias=0)
KV = {"f32": K.ML_F32, "f16": K.ML_F16, "q8": K.ML_Q8_0}


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


@pytest.mark.parametrize("hd,nh,nkv,normed", [(128, 32, 8, True), (64, 4, 2, True), (256, 3, 1, True),
                                             (128, 4, 4, False), (2, 1, 1, True)])
def test_heads_norm_rope(hd, nh, nkv, normed):
    """each head: k_scalar.c:59-64's rmsnorm with the head weight, then
    k_scalar.c:79-94's rotation by the tables' row *pos"""
    rng = np.random.default_rng(hd + nh)
    q = (rng.standard_normal(nh * hd) * 3).astype(np.float32)
    k = (rng.standard_normal(nkv * hd) * 3).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    P, pos = 40, 33
    ang = rng.uniform(-3, 3, (P, hd // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    eps = np.float32(1e-6)
    wq, wk = q.copy(), k.copy()
    if normed:
        for h in range(nh):
            seg = wq[h * hd:(h + 1) * hd].copy()
            oracle.kro_rmsnorm(wq[h * hd:].ctypes.data, seg.ctypes.data, qw.ctypes.data, hd, eps)
        for h in range(nkv):
            seg = wk[h * hd:(h + 1) * hd].copy()
            oracle.kro_rmsnorm(wk[h * hd:].ctypes.data, seg.ctypes.data, kw.ctypes.data, hd, eps)
    c0, s0 = np.ascontiguousarray(cs[pos]), np.ascontiguousarray(sn[pos])
    oracle.kro_rope(wq.ctypes.data, wk.ctypes.data, c0.ctypes.data, s0.ctypes.data, hd, nh, nkv)
    bufs = [K.DevBuf.of(a) for a in (q, k, qw, kw, cs, sn, np.array([pos], np.int32))]
    qb, kb, qwb, kwb, cb, sb, pb = bufs
    K.hip.krh_heads_norm_rope(qb.ptr, kb.ptr, qwb.ptr if normed else None, kwb.ptr if normed else None, cb.ptr,
                              sb.ptr, hd, nh, nkv, eps, pb.ptr)
    ok()
    assert np.array_equal(bits(qb.get(np.float32, nh * hd)), bits(wq))
    assert np.array_equal(bits(kb.get(np.float32, nkv * hd)), bits(wk))
    for b in bufs:
        b.free()


def test_tanhf_exhaustive():
    """the device tanhf (and the expm1f under it) equals the host C library's
    on every float32 input"""
    n = 1 << 26
    y = K.DevBuf(4 * n)
    try:
        for lo in range(0, 1 << 32, n):
            K.hip.krh_tanhf_range(y.ptr, lo, n)
            ok()
            got = y.get(np.float32, n)
            assert oracle.kro_tanhf_check_range(lo, got.ctypes.data, n, 16) == 0, hex(lo)
    finally:
        y.free()


@pytest.mark.parametrize("n", [1, 333, 14336])
def test_gelu_softcap_ops(n):
    """the op table's gelu_mul and softcap kernels against the oracle's
    (pinned to the reference's scalar kernels)"""
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    want = g.copy()
    oracle.kro_gelu_mul(want.ctypes.data, u.ctypes.data, n)
    gb, ub = K.DevBuf.of(g), K.DevBuf.of(u)
    K.hip.krh_gelu_mul(gb.ptr, ub.ptr, n)
    ok()
    assert np.array_equal(bits(gb.get(np.float32, n)), bits(want))
    x = (rng.standard_normal(2 * n) * 40).astype(np.float32)
    want = x.copy()
    oracle.kro_softcap_rows(want.ctypes.data, n, 2, n, 30.0)
    xb = K.DevBuf.of(x)
    K.hip.krh_softcap_rows(xb.ptr, n, 2, n, 30.0)
    ok()
    assert np.array_equal(bits(xb.get(np.float32, 2 * n)), bits(want))
    for b in (gb, ub, xb):
        b.free()


def test_store_rows_f32():
    n, rows, pos = 640, 9, 7
    k = np.arange(n, dtype=np.float32)
    v = -k
    kc, vc = K.DevBuf.of(np.zeros(rows * n, np.float32)), K.DevBuf.of(np.zeros(rows * n, np.float32))
    kb, vb, pb = K.DevBuf.of(k), K.DevBuf.of(v), K.DevBuf.of(np.array([pos], np.int32))
    K.hip.krh_store_rows_f32(kc.ptr, vc.ptr, kb.ptr, vb.ptr, n, pb.ptr)
    ok()
    want = np.zeros((rows, n), np.float32)
    want[pos] = k
    assert np.array_equal(kc.get(np.float32, rows * n).reshape(rows, n), want)
    want[pos] = v
    assert np.array_equal(vc.get(np.float32, rows * n).reshape(rows, n), want)
    for b in (kc, vc, kb, vb, pb):
        b.free()


@pytest.mark.parametrize("kv", sorted(KV))
@pytest.mark.parametrize("name", sorted(FAMILY) + sorted(VARIANTS))
def test_family_model_matches_reference(name, kv, workdir):
    """logits of every prompt position (ml_run --dump-logits --kv) and greedy
    ids (ml_run -T 0 --kv) on a generated model of the family"""
    path = os.path.join(workdir, "fam_" + name + ".mlb")
    if not os.path.exists(path):
        K.gen_mlb(path, **(FAMILY.get(name) or VARIANTS[name]))
    m = K.Model(path)
    s = K.State(m, KV[kv])
    V = m.cfg.vocab
    toks = [int(t) for t in np.random.default_rng(5).integers(1, V, 12)]
    dump = path + "." + kv + ".logits"
    print("family", name, kv, flush=True)
    O.ref_ml_run(path, toks, len(toks), dump=dump, extra=("--kv", kv))
    want = np.fromfile(dump, dtype=np.float32).reshape(len(toks), V)
    got = np.empty((len(toks), V), dtype=np.float32)
    s.prefill(toks, 0, logits=got)
    assert np.array_equal(bits(got), bits(want))
    s.close()
    s = K.State(m, KV[kv])
    steps = min(m.cfg.max_seq, 8 + 80)
    want_ids, _ = O.ref_ml_run(path, toks[:8], steps, extra=("--kv", kv))
    got_ids, _, _ = s.generate(toks[:8], steps)
    assert np.array_equal(got_ids, want_ids)
    s.close()
    m.close()


@pytest.mark.parametrize("kv", sorted(KV))
@pytest.mark.parametrize("name", ["qk_norm_bias_gqa", "qk_post_norms_f16", "window_local_rope_layers",
                                  "gelu_softcap_gemma2", "gelu_post_qk_gemma3", "gemma2_wide_heads"])
def test_family_batched_prefill(name, kv, workdir):
    """the families' batched prefill (token_stage's per-token stages as row
    launches, model/transformer.c:324-365) over a prompt that passes the
    sliding windows, in one step, in ragged steps of 7 and token by token:
    every position's logits equal ml_run --dump-logits"""
    spec = FAMILY.get(name) or VARIANTS[name]
    path = os.path.join(workdir, "fam_" + name + ".mlb")
    if not os.path.exists(path):
        K.gen_mlb(path, **spec)
    m = K.Model(path)
    V = m.cfg.vocab
    n = min(m.cfg.max_seq - 2, 90)
    toks = [int(t) for t in np.random.default_rng(9).integers(1, V, n)]
    dump = path + "." + kv + ".long.logits"
    print("family batched", name, kv, n, flush=True)
    O.ref_ml_run(path, toks, n, dump=dump, extra=("--kv", kv))
    want = np.fromfile(dump, dtype=np.float32).reshape(n, V)
    for batch in (0, 7, 1):
        s = K.State(m, KV[kv])
        if batch:
            s.set_batch(batch)
        got = np.empty((n, V), dtype=np.float32)
        s.prefill(toks, 0, logits=got)
        s.close()
        bad = np.nonzero(~np.all(bits(got) == bits(want), axis=1))[0]
        assert bad.size == 0, "batch %d: positions %s differ" % (batch, bad[:8])
    m.close()
