"""The .mlb loader (isa-lm_amd/host/kr_mlb.c) against the reference's own
loader (ml_model_load, model/mlb.c, in oracle/_ref/libkrafla_ref_scalar.so):
valid models of every layout load with the same configuration, and patched
headers, flag bytes and tensor bytes and truncated files give the same status
as the reference (the way tests/test_load.c:76-300 patches files). CPU only."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

import krafla as K
from oracle_lib import ref

pytestmark = pytest.mark.skipif(ref is None, reason="oracle/_ref not built (needs /root/reference at build time)")

OK, IO, FORMAT, SHAPE = 0, 1, 2, 3
MODEL_BYTES = 1 << 14   # ml_model is a few hundred bytes: room to spare

BASES = {
    "q8_f32": dict(K.CONFIGS["stories15m_q8"], dim=64, n_layers=2, n_heads=4, n_kv_heads=2, hidden_dim=96,
                   vocab=40, max_seq=32),
    "q4mix_f16_tied_bias": dict(K.CONFIGS["qwen05b_mixed"], dim=64, n_layers=2, n_heads=4, n_kv_heads=2,
                                hidden_dim=96, vocab=50, max_seq=32),
    "q8_f16_llama3": dict(K.CONFIGS["llama8b_q8"], dim=128, n_layers=1, n_heads=4, n_kv_heads=1, hidden_dim=64,
                          vocab=33, max_seq=16, rope_type=K.ML_ROPE_LLAMA3, rope_factor=8.0,
                          rope_low_freq_factor=1.0, rope_high_freq_factor=4.0, rope_orig_max_seq=64),
    "family_flags": dict(K.CONFIGS["stories15m_q8"], dim=64, n_layers=3, n_heads=2, n_kv_heads=1, hidden_dim=64,
                         vocab=20, max_seq=16, qk_norm=1, post_norms=1, act=1, sliding_window=4,
                         layer_sliding=0b101, layer_local=0b010, rope_local_theta=1e4, embed_scale=8.0,
                         attn_softcap=50.0, final_softcap=30.0),
}


def ref_load(path):
    buf = C.create_string_buffer(MODEL_BYTES)
    st = ref.ml_model_load(buf, path.encode())
    cfg = bytes(buf.raw[:C.sizeof(K.MlConfig)])
    if st == OK:
        ref.ml_model_free(buf)
    return st, cfg


def our_load(path):
    p = C.c_void_p()
    st = K.host.kr_model_load(C.byref(p), path.encode())
    cfg = None
    if st == OK:
        cfg = bytes(C.string_at(C.addressof(K.host.kr_model_config(p).contents), C.sizeof(K.MlConfig)))
        K.host.kr_model_free(p)
    return st, cfg


@pytest.fixture(scope="module")
def bases(tmp_path_factory):
    d = tmp_path_factory.mktemp("loader")
    out = {}
    for name, spec in BASES.items():
        path = str(d / (name + ".mlb"))
        K.gen_mlb(path, **spec)
        with open(path, "rb") as f:
            out[name] = f.read()
    return d, out


def check_same(d, name, data):
    path = str(d / "case.mlb")
    with open(path, "wb") as f:
        f.write(data)
    want, wcfg = ref_load(path)
    got, gcfg = our_load(path)
    assert got == want, "%s: status %d, the reference's %d" % (name, got, want)
    if want == OK:
        assert gcfg == wcfg, "%s: configuration differs" % name
    return got


def set_u32(data, off, v):
    b = bytearray(data)
    b[off:off + 4] = struct.pack("<I", v & 0xFFFFFFFF)
    return bytes(b)


def set_f32(data, off, v):
    b = bytearray(data)
    b[off:off + 4] = struct.pack("<f", v)
    return bytes(b)


def test_valid_models_load_alike(bases):
    d, data = bases
    for name, blob in data.items():
        assert check_same(d, name, blob) == OK


NAN, INF = float("nan"), float("inf")
HEADER_CASES = [
    ("magic", lambda b: b"MLB2" + b[4:]), ("magic case", lambda b: b"mlb1" + b[4:]),
    ("version 0", lambda b: set_u32(b, 4, 0)), ("version 2", lambda b: set_u32(b, 4, 2)),
] + [
    ("%s = %d" % (n, v), (lambda o, v: lambda b: set_u32(b, o, v))(o, v))
    for n, o, vals in [("dim", 8, [0, 33, 65537, 1 << 31]), ("n_layers", 12, [0, 65537]),
                       ("n_heads", 16, [0, 3, 65537]), ("n_kv_heads", 20, [0, 3, 65537]),
                       ("hidden_dim", 24, [0, 40, 65537]), ("vocab", 28, [0, 2, (1 << 24) + 1]),
                       ("max_seq", 32, [0, (1 << 24) + 1]), ("wtype", 44, [0, 3, 0xFFFFFFFF]),
                       ("shared", 48, [7]), ("rope_type", 52, [4, 0xFFFFFFFF]),
                       ("q8_mask", 72, [128, 0x80000000, 1]), ("qkv_bias", 76, [2]),
                       ("head_dim", 80, [63, 65537, 4096, 2]), ("qk_norm", 84, [2]),
                       ("sliding_window", 92, [(1 << 24) + 1, 1 << 24]), ("layer_flags", 96, [2]),
                       ("act", 104, [2]), ("post_norms", 108, [2]), ("scale_f16", 120, [2, 1, 0])]
    for v in vals
] + [
    ("%s = %r" % (n, v), (lambda o, v: lambda b: set_f32(b, o, v))(o, v))
    for n, o, vals in [("rope_theta", 36, [0.0, -1.0, NAN, INF]), ("norm_eps", 40, [-1e-5, NAN, INF]),
                       ("rope_attn_factor", 88, [1.0]),
                       ("rope_local_theta", 100, [-1.0, NAN, 1e30, 9.99e29]),
                       ("embed_scale", 112, [-1.0, NAN, 1e6, 999999.9, -0.0]),
                       ("attn_scale", 116, [1e6, INF, -0.0]), ("attn_softcap", 124, [-1.0, 1e6, INF]),
                       ("final_softcap", 128, [NAN, 2.5])]
    for v in vals
]


def rope_case(rtype, factor, lo, hi, orig, attn=0.0):
    def f(b):
        b = set_u32(b, 52, rtype)
        b = set_f32(b, 56, factor)
        b = set_f32(b, 60, lo)
        b = set_f32(b, 64, hi)
        b = set_u32(b, 68, orig)
        return set_f32(b, 88, attn)
    return f


ROPE_CASES = [
    ("llama3 ok", rope_case(1, 8.0, 1.0, 4.0, 64)), ("llama3 factor 0", rope_case(1, 0.0, 1.0, 4.0, 64)),
    ("llama3 factor 1e6", rope_case(1, 1e6, 1.0, 4.0, 64)), ("llama3 lo 0", rope_case(1, 8.0, 0.0, 4.0, 64)),
    ("llama3 hi = lo", rope_case(1, 8.0, 2.0, 2.0, 64)), ("llama3 orig 0", rope_case(1, 8.0, 1.0, 4.0, 0)),
    ("llama3 with attn factor", rope_case(1, 8.0, 1.0, 4.0, 64, 1.0)),
    ("linear ok", rope_case(2, 4.0, 0.0, 0.0, 0)), ("linear factor NaN", rope_case(2, NAN, 0.0, 0.0, 0)),
    ("yarn ok", rope_case(3, 4.0, 32.0, 1.0, 64, 1.2)), ("yarn no attn factor", rope_case(3, 4.0, 32.0, 1.0, 64)),
    ("yarn attn factor 1e3", rope_case(3, 4.0, 32.0, 1.0, 64, 1e3)),
    ("yarn beta_fast <= beta_slow", rope_case(3, 4.0, 1.0, 1.0, 64, 1.0)),
    ("yarn beta_slow 0", rope_case(3, 4.0, 32.0, 0.0, 64, 1.0)),
    ("yarn orig 0", rope_case(3, 4.0, 32.0, 1.0, 0, 1.0)),
]


@pytest.mark.parametrize("base", sorted(BASES))
def test_header_patches(bases, base):
    d, data = bases
    statuses = set()
    for name, patch in HEADER_CASES + ROPE_CASES:
        statuses.add(check_same(d, "%s: %s" % (base, name), patch(data[base])))
    assert {OK, FORMAT, SHAPE} <= statuses


@pytest.mark.parametrize("base", sorted(BASES))
def test_header_two_faults(bases, base):
    """two patched fields whose single faults give different statuses: the
    reference interleaves field ranges with the rules between fields
    (model/mlb.c:80-157), so the status is that of the first fault in its
    order; every such pair of the single-field cases, applied together"""
    d, data = bases
    blob = data[base]
    single = [(name, patch, check_same(d, "%s: %s" % (base, name), patch(blob)))
              for name, patch in HEADER_CASES + ROPE_CASES]
    bad = [(n, p, st) for n, p, st in single if st != OK]
    pairs = 0
    for i, (na, pa, sa) in enumerate(bad):
        for nb, pb, sb in bad[i + 1:]:
            if sa != sb:
                check_same(d, "%s: %s + %s" % (base, na, nb), pb(pa(blob)))
                pairs += 1
    assert pairs > 100
    # the examples that separate the orders: a SHAPE fault before a later
    # FORMAT one, and a FORMAT fault before a later SHAPE one
    assert check_same(d, base + ": dim 40, rope_theta 0", set_f32(set_u32(blob, 8, 40), 36, 0.0)) == SHAPE
    if BASES[base]["wtype"] == K.ML_Q8_0:
        assert check_same(d, base + ": q8_mask 1, head_dim 65537", set_u32(set_u32(blob, 72, 1), 80, 65537)) == FORMAT


def align64(n):
    return (n + 63) // 64 * 64


def body_layout(spec):
    """(name, offset, bytes, q8) of every array, from the specification's
    list (docs/file-format.md:81-101), for the generator's spec"""
    dim, L, nh, nkv, hid, V = (spec[k] for k in ("dim", "n_layers", "n_heads", "n_kv_heads", "hidden_dim", "vocab"))
    hd = dim // nh
    qd, kvd = hd * nh, hd * nkv
    wq8 = spec["wtype"] == K.ML_Q8_0
    mask = spec["q8_mask"] if not wq8 else 0
    sb = 2 if spec["scale_f16"] else 4
    shared = spec["shared"]
    out = []
    off = 256
    if spec.get("layer_sliding") or spec.get("layer_local"):
        out.append(("flags", off, L, False))
        off = align64(off + L)

    def arr(name, n, q8=False):
        nonlocal off
        out.append((name, off, n, q8))
        off = align64(off + n)

    def mat(name, rows, cols, bits):
        q8 = wq8 or bool(mask & bits)
        arr(name + ".q", rows * cols if q8 else rows * cols // 2, q8)
        arr(name + ".d", rows * cols // 32 * sb)

    mat("tok_emb", V, dim, 1 | (2 if shared else 0))
    for layer in range(L):
        arr("attn_norm", 4 * dim)
        mat("wq", qd, dim, 4)
        mat("wk", kvd, dim, 4)
        mat("wv", kvd, dim, 8)
        mat("wo", dim, qd, 16)
        if spec["qkv_bias"]:
            arr("bq", 4 * qd)
            arr("bk", 4 * kvd)
            arr("bv", 4 * kvd)
        if spec["qk_norm"]:
            arr("q_norm", 4 * hd)
            arr("k_norm", 4 * hd)
        arr("ffn_norm", 4 * dim)
        mat("w1", hid, dim, 32)
        mat("w2", dim, hid, 64)
        mat("w3", hid, dim, 32)
        if spec["post_norms"]:
            arr("post_attn_norm", 4 * dim)
            arr("post_ffn_norm", 4 * dim)
    arr("final_norm", 4 * dim)
    if not shared:
        mat("wcls", V, dim, 2)
    return out


@pytest.mark.parametrize("base", sorted(BASES))
def test_body_patches_and_truncation(bases, base):
    d, data = bases
    blob = data[base]
    layout = body_layout(BASES[base])
    end = layout[-1][1] + layout[-1][2]
    assert end <= len(blob) <= align64(end)   # the layout above is the file's
    cases = []
    for name, off, n, q8 in layout:
        b = bytearray(blob)
        b[off] = 0x80   # a Q8 quant of -128 (rejected), or any other byte (accepted)
        cases.append(("0x80 at the start of " + name, bytes(b)))
        b = bytearray(blob)
        b[off + n - 1] = 0x80
        cases.append(("0x80 at the end of " + name, bytes(b)))
    for name, off, n, q8 in layout[::3] + layout[-2:]:
        cases.append(("cut inside " + name, blob[:off + n // 2]))
        cases.append(("cut after " + name, blob[:off + n]))
    for n in (0, 1, 100, 255, 256, 257, len(blob) - 1, end):
        cases.append(("cut to %d bytes" % n, blob[:n]))
    cases.append(("padding after the last array", blob[:end] + bytes(align64(end) - end + 64)))
    if base == "family_flags":
        for bit in (4, 0x80):
            b = bytearray(blob)
            b[257] |= bit
            cases.append(("flag bit 0x%x" % bit, bytes(b)))
        cases.append(("local RoPE flag without rope_local_theta", set_f32(blob, 100, 0.0)))
    seen = set()
    for name, patched in cases:
        seen.add(check_same(d, "%s: %s" % (base, name), patched))
    assert FORMAT in seen and OK in seen


def test_missing_and_unreadable(tmp_path):
    for path in (str(tmp_path / "absent.mlb"), str(tmp_path)):
        want, _ = ref_load(path)
        got, _ = our_load(path)
        assert got == want == IO or (got == want), (path, got, want)
