"""ctypes access to the checkers: the oracle's C restatement
(oracle/_build/liboracle.so) and the reference's own scalar build
(oracle/_ref/libkrafla_ref_scalar.so, oracle/_ref/<isa>/ml_run). Test
infrastructure only."""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "_build", "liboracle.so")
REF_DIR = os.path.join(ROOT, "oracle", "_ref")
REF_SO = os.path.join(REF_DIR, "libkrafla_ref_scalar.so")

import krafla as K  # noqa: E402  (tests/conftest.py puts the package on sys.path)

_P = C.c_void_p


def _lib(path):
    if not os.path.exists(path):
        raise RuntimeError("%s missing: run __graft_entry__.build()" % path)
    return C.CDLL(path)


oracle = _lib(ORACLE_SO)
ref = _lib(REF_SO) if os.path.exists(REF_SO) else None

KERNELS = {
    "matvec_q8": [_P, _P, _P, C.c_int, C.c_int], "matvec_q4": [_P, _P, _P, C.c_int, C.c_int],
    "quantize_q8": [_P, _P, C.c_int], "rmsnorm": [_P, _P, _P, C.c_int, C.c_float],
    "softmax": [_P, C.c_int], "rope": [_P, _P, _P, _P, C.c_int, C.c_int, C.c_int],
    "silu_mul": [_P, _P, C.c_int], "add": [_P, _P, C.c_int],
    "dot_f32": [_P, _P, _P, C.c_size_t, C.c_int, C.c_int, C.c_float],
    "axpy_f32": [_P, _P, _P, C.c_size_t, C.c_int, C.c_int],
}
for name, args in KERNELS.items():
    getattr(oracle, "kro_" + name).argtypes = args
    if ref is not None:
        getattr(ref, "ml_k_%s_scalar" % name).argtypes = args
oracle.kro_expf.restype = C.c_float
oracle.kro_expf.argtypes = [C.c_float]
oracle.kro_expf_mismatches.restype = C.c_uint64
oracle.kro_expf_mismatches.argtypes = [C.c_uint64, C.c_uint64, C.c_int]
oracle.kro_expf_check.restype = C.c_uint64
oracle.kro_expf_check.argtypes = [_P, _P, C.c_size_t]
oracle.kro_expf_check_range.restype = C.c_uint64
oracle.kro_expf_check_range.argtypes = [C.c_uint64, _P, C.c_size_t, C.c_int]
oracle.kro_tanhf.restype = C.c_float
oracle.kro_tanhf.argtypes = [C.c_float]
oracle.kro_tanhf_mismatches.restype = C.c_uint64
oracle.kro_tanhf_mismatches.argtypes = [C.c_uint64, C.c_uint64, C.c_int]
oracle.kro_gelu_mul.argtypes = [_P, _P, C.c_int]
oracle.kro_tanhf_check_range.restype = C.c_uint64
oracle.kro_tanhf_check_range.argtypes = [C.c_uint64, _P, C.c_size_t, C.c_int]
oracle.kro_softcap_rows.argtypes = [_P, C.c_size_t, C.c_int, C.c_int, C.c_float]
if ref is not None:
    ref.ml_k_gelu_mul_scalar.argtypes = [_P, _P, C.c_int]
    ref.ml_softcap_rows.argtypes = [_P, C.c_size_t, C.c_int, C.c_int, C.c_float]
oracle.kro_f32_to_f16.restype = C.c_uint16
oracle.kro_f32_to_f16.argtypes = [C.c_float]
oracle.kro_f32_to_f16_range.argtypes = [_P, C.c_uint32, C.c_size_t]
oracle.kro_f32_to_f16_mismatches.restype = C.c_uint64
oracle.kro_f32_to_f16_mismatches.argtypes = [C.c_uint64, C.c_uint64, C.c_int]
KV_KERNELS = {
    "dot_f16": [_P, _P, _P, C.c_size_t, C.c_int, C.c_int, C.c_float],
    "axpy_f16": [_P, _P, _P, C.c_size_t, C.c_int, C.c_int],
    "dot_q8": [_P, _P, C.c_float, _P, _P, C.c_size_t, C.c_size_t, C.c_int, C.c_int, C.c_float],
    "axpy_q8": [_P, _P, _P, _P, C.c_size_t, C.c_size_t, C.c_int, C.c_int],
}
for name, args in KV_KERNELS.items():
    getattr(oracle, "kro_" + name).argtypes = args
    if ref is not None:
        getattr(ref, "ml_k_%s_scalar" % name).argtypes = args
oracle.kro_quantize_row.argtypes = [_P, _P, _P, C.c_int]
oracle.kro_state_new_kv.argtypes = [C.POINTER(_P), _P, C.c_int]
oracle.kro_state_cache.restype = _P
oracle.kro_state_cache.argtypes = [_P, C.c_char_p]
oracle.kro_f16_to_f32.restype = C.c_float
oracle.kro_f16_to_f32.argtypes = [C.c_uint16]
oracle.kro_dequant_row.argtypes = [_P, _P, C.c_int]
oracle.kro_quantize_row_q4.argtypes = [_P, _P, _P, C.c_int]
oracle.kro_block_dots.argtypes = [_P, _P, _P, C.c_int, C.c_int]
oracle.kro_argmax.restype = C.c_int
oracle.kro_argmax.argtypes = [_P, C.c_int]
oracle.kro_attention.argtypes = [_P, _P, _P, _P, _P, C.c_int]
oracle.kro_model_open.argtypes = [C.POINTER(_P), C.c_char_p]
oracle.kro_model_config.restype = C.POINTER(K.MlConfig)
oracle.kro_model_config.argtypes = [_P]
oracle.kro_model_close.argtypes = [_P]
oracle.kro_state_new.argtypes = [C.POINTER(_P), _P]
oracle.kro_state_free.argtypes = [_P]
oracle.kro_forward.argtypes = [_P, C.c_int, C.c_int, _P]
oracle.kro_prefill.argtypes = [_P, _P, C.c_int, C.c_int, _P]
oracle.kro_generate.argtypes = [_P, _P, C.c_int, C.c_int, _P]
oracle.kro_state_buffer.restype = C.POINTER(C.c_float)
oracle.kro_state_buffer.argtypes = [_P, C.c_char_p]
oracle.kro_state_x.restype = C.POINTER(C.c_float)
oracle.kro_state_x.argtypes = [_P]
if ref is not None:
    ref.ml_quantize_row.argtypes = [_P, _P, _P, C.c_int]
    ref.ml_f32_to_f16.restype = C.c_uint16
    ref.ml_f32_to_f16.argtypes = [C.c_float]
    ref.ml_dequant_row.argtypes = [_P, _P, C.c_int]
    ref.ml_quantize_row_q4.argtypes = [_P, _P, _P, C.c_int]


KvLayer = K.MlKvLayer   # ops/ops.h:16-22


def qtensor(q, d, rows, cols, typ):
    """an ml_qtensor over numpy arrays q (int8/uint8) and d (float32)"""
    return K.MlQTensor(q.ctypes.data, d.ctypes.data, rows, cols, typ, None, None, None, 0)


def qact(q, d):
    return K.MlQAct(q.ctypes.data, d.ctypes.data, len(q))


def quantize(x):
    """Q8_0 of x with the oracle (int8 quants, f32 scales)"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.zeros(len(x), dtype=np.int8)
    d = np.zeros(len(x) // 32, dtype=np.float32)
    a = qact(q, d)
    oracle.kro_quantize_q8(C.byref(a), x.ctypes.data, len(x))
    return q, d


class OracleModel:
    def __init__(self, path, kv_type=K.ML_F32):
        self.m = _P()
        st = oracle.kro_model_open(C.byref(self.m), path.encode())
        assert st == 0, "oracle cannot open %s (%d)" % (path, st)
        self.cfg = oracle.kro_model_config(self.m).contents
        self.s = _P()
        assert oracle.kro_state_new_kv(C.byref(self.s), self.m, kv_type) == 0

    def cache(self, name, count, dtype):
        """the F16 / Q8 cache array by name ("kh", "vh", "kq", "vq", "kd", "vd")"""
        p = oracle.kro_state_cache(self.s, name.encode())
        assert p, name
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(np.ctypeslib.as_ctypes_type(dtype))), shape=(count,)).copy()

    def forward(self, tok, pos):
        out = np.empty(self.cfg.vocab, dtype=np.float32)
        assert oracle.kro_forward(self.s, tok, pos, out.ctypes.data) == 0
        return out

    def prefill(self, toks, pos0, logits=False):
        t = np.ascontiguousarray(toks, dtype=np.int32)
        out = np.empty((len(t), self.cfg.vocab), dtype=np.float32) if logits else None
        assert oracle.kro_prefill(self.s, t.ctypes.data, len(t), pos0,
                                  out.ctypes.data if out is not None else None) == 0
        return out

    def generate(self, prompt, steps):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(steps + len(p) + 2, dtype=np.int32)
        n = oracle.kro_generate(self.s, p.ctypes.data, len(p), steps, out.ctypes.data)
        assert n >= 0
        return out[:n].copy()

    def generate_sampled(self, sampler, prompt, steps):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(steps + len(p) + 2, dtype=np.int32)
        n = oracle.kro_generate_sampled(self.s, sampler.s, p.ctypes.data, len(p), steps, out.ctypes.data)
        assert n >= 0
        return out[:n].copy()

    def buffer(self, name, count):
        p = oracle.kro_state_buffer(self.s, name.encode())
        return np.ctypeslib.as_array(p, shape=(count,)).copy()

    def close(self):
        oracle.kro_state_free(self.s)
        oracle.kro_model_close(self.m)


# ml_sampler_opts (model/sampler.h:9-16): kro_sampler_opts and
# krh_sampler_opts share its layout
SamplerOpts = K.SamplerOpts
sampler_opts = K.sampler_opts


class RefSampler(C.Structure):
    """ml_sampler (model/sampler.h:18-27)"""
    _fields_ = [("o", SamplerOpts), ("rng", C.c_uint64), ("vocab", C.c_int), ("probs", _P), ("cand", _P),
                ("recent", _P), ("n_recent", C.c_int), ("recent_at", C.c_int), ("mark", _P), ("stamp", C.c_int)]


oracle.kro_sampler_new.argtypes = [_P, C.c_int, C.POINTER(SamplerOpts)]
oracle.kro_sampler_free.argtypes = [_P]
oracle.kro_sampler_accept.argtypes = [_P, C.c_int]
oracle.kro_sample.argtypes = [_P, _P, C.c_int]
oracle.kro_sampler_rng.restype = C.c_uint64
oracle.kro_sampler_rng.argtypes = [_P]
oracle.kro_generate_sampled.argtypes = [_P, _P, _P, C.c_int, C.c_int, _P]
if ref is not None:
    ref.ml_sampler_init.argtypes = [C.POINTER(RefSampler), C.c_int, C.POINTER(SamplerOpts)]
    ref.ml_sampler_accept.argtypes = [C.POINTER(RefSampler), C.c_int]
    ref.ml_sample.argtypes = [C.POINTER(RefSampler), _P, C.c_int]
    ref.ml_sampler_free.argtypes = [C.POINTER(RefSampler)]


class OracleSampler:
    def __init__(self, vocab, opts):
        self.s = _P()
        assert oracle.kro_sampler_new(C.byref(self.s), vocab, C.byref(opts)) == 0

    def accept(self, tok):
        oracle.kro_sampler_accept(self.s, int(tok))

    def sample(self, logits):
        """the id; logits (float32, modified in place as the reference does)"""
        assert logits.dtype == np.float32 and logits.flags.c_contiguous
        return oracle.kro_sample(self.s, logits.ctypes.data, len(logits))

    @property
    def rng(self):
        return oracle.kro_sampler_rng(self.s)

    def close(self):
        oracle.kro_sampler_free(self.s)


class ReferenceSampler:
    """the reference's own ml_sampler (oracle/_ref/libkrafla_ref_scalar.so)"""

    def __init__(self, vocab, opts):
        self.s = RefSampler()
        assert ref.ml_sampler_init(C.byref(self.s), vocab, C.byref(opts)) == 0

    def accept(self, tok):
        ref.ml_sampler_accept(C.byref(self.s), int(tok))

    def sample(self, logits):
        assert logits.dtype == np.float32 and logits.flags.c_contiguous
        return ref.ml_sample(C.byref(self.s), logits.ctypes.data, len(logits))

    @property
    def rng(self):
        return self.s.rng

    def close(self):
        ref.ml_sampler_free(C.byref(self.s))


def ref_ml_run(model, tokens, steps, threads=1, dump=None, isa="scalar", timeout=600, extra=()):
    """the reference's own ml_run (built from its sources into oracle/_ref;
    isa "hip": over this repository's op-table binding): greedy ids it
    prints, or the logits it dumps; with its stderr"""
    exe = os.path.join(REF_DIR, isa, "ml_run")
    cmd = [exe, model, "--tokens", ",".join(str(int(t)) for t in tokens), "-n", str(steps), "-T", "0",
           "-t", str(threads)] + list(extra)
    if dump:
        cmd += ["--dump-logits", dump]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError("ml_run failed (%d): %s" % (r.returncode, r.stderr))
    ids = np.array([int(v) for v in r.stdout.split()], dtype=np.int32)
    return ids, r.stderr
