"""ctypes binding of libkrafla.so / libkrafla_hip.so for tests and bench.py.

The libraries are the product; this module only loads them and wraps their C
ABI (include/krafla.h, include/krafla_hip.h). There is no fallback: if the
built libraries are missing, importing the binding raises.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_HIP = os.path.join(HERE, "libkrafla_hip.so")
LIB_HOST = os.path.join(HERE, "libkrafla.so")

ML_OK, ML_E_IO, ML_E_FORMAT, ML_E_SHAPE, ML_E_NOMEM, ML_E_ISA = range(6)
ML_F32, ML_Q8_0, ML_Q4_0, ML_F16 = 0, 1, 2, 3
ML_ROPE_NONE, ML_ROPE_LLAMA3, ML_ROPE_LINEAR, ML_ROPE_YARN = 0, 1, 2, 3
ML_ACT_SILU, ML_ACT_GELU_TANH = 0, 1
MATH_EXPF, MATH_SQRT, MATH_DIV, MATH_RMS_INV = range(4)
Q8M_EMB, Q8M_CLS, Q8M_QK, Q8M_V, Q8M_O, Q8M_UP, Q8M_DOWN = 1, 2, 4, 8, 16, 32, 64


class MlKvLayer(C.Structure):
    """ml_kv_layer (ops/ops.h:16-22): one layer's cache view, device pointers"""
    _fields_ = [("k", C.c_void_p), ("v", C.c_void_p), ("kq", C.c_void_p), ("vq", C.c_void_p), ("kd", C.c_void_p),
                ("vd", C.c_void_p), ("window", C.c_int), ("kh", C.c_void_p), ("vh", C.c_void_p)]


class MlConfig(C.Structure):
    """model/mlb.h:9-40"""
    _fields_ = [(n, C.c_int) for n in ("dim", "n_layers", "n_heads", "n_kv_heads", "hidden_dim", "vocab",
                                       "max_seq", "head_dim", "kv_dim", "q_dim")] + [
        ("rope_theta", C.c_float), ("norm_eps", C.c_float), ("wtype", C.c_int), ("q8_mask", C.c_uint),
        ("qkv_bias", C.c_int), ("qk_norm", C.c_int), ("sliding_window", C.c_int), ("layer_flags", C.c_int),
        ("rope_local_theta", C.c_float), ("act", C.c_int), ("post_norms", C.c_int), ("embed_scale", C.c_float),
        ("attn_scale", C.c_float), ("scale_f16", C.c_int), ("attn_softcap", C.c_float),
        ("final_softcap", C.c_float), ("rope_type", C.c_int), ("rope_orig_max_seq", C.c_int),
        ("rope_factor", C.c_float), ("rope_low_freq_factor", C.c_float), ("rope_high_freq_factor", C.c_float),
        ("rope_attn_factor", C.c_float)]


class MlQTensor(C.Structure):
    """core/ml.h:71-83"""
    _fields_ = [("q", C.c_void_p), ("d", C.c_void_p), ("rows", C.c_int), ("cols", C.c_int), ("type", C.c_uint8),
                ("pq", C.c_void_p), ("pd", C.c_void_p), ("dh", C.c_void_p), ("pd16", C.c_uint8)]


class MlQAct(C.Structure):
    _fields_ = [("q", C.c_void_p), ("d", C.c_void_p), ("n", C.c_int)]


class KrhMat(C.Structure):
    _fields_ = [("q", C.c_void_p), ("d", C.c_void_p), ("rows", C.c_int), ("cols", C.c_int), ("type", C.c_int),
                ("d16", C.c_int)]


class GenSpec(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("dim", "n_layers", "n_heads", "n_kv_heads", "hidden_dim", "vocab",
                                       "max_seq")] + [
        ("rope_theta", C.c_float), ("norm_eps", C.c_float), ("wtype", C.c_int), ("q8_mask", C.c_uint),
        ("shared", C.c_int), ("qkv_bias", C.c_int), ("scale_f16", C.c_int), ("rope_type", C.c_int),
        ("rope_factor", C.c_float), ("rope_low_freq_factor", C.c_float), ("rope_high_freq_factor", C.c_float),
        ("rope_orig_max_seq", C.c_int), ("std", C.c_float), ("seed", C.c_uint64), ("threads", C.c_int), ("device", C.c_int),
        ("qk_norm", C.c_int), ("post_norms", C.c_int), ("sliding_window", C.c_int), ("layer_sliding", C.c_uint),
        ("layer_local", C.c_uint), ("rope_local_theta", C.c_float), ("rope_attn_factor", C.c_float),
        ("act", C.c_int), ("embed_scale", C.c_float), ("attn_softcap", C.c_float), ("final_softcap", C.c_float)]


# The workloads, by name. Shapes and quantization as the benchmark configs
# state them; assumptions where they are silent: max_seq 1024 for the
# Qwen2.5-0.5B shape, Llama-3.2's rope scaling (factor 32, 1, 4, 8192) and
# tied classifier for the 1B shape, f16 scales and max_seq 4096 for the 8B
# shape (its "about 8.5 GB" is the f16-scale size).
def _spec(**kw):
    base = dict(rope_theta=1e4, norm_eps=1e-5, wtype=ML_Q8_0, q8_mask=0, shared=0, qkv_bias=0, scale_f16=0,
                rope_type=ML_ROPE_NONE, rope_factor=0.0, rope_low_freq_factor=0.0, rope_high_freq_factor=0.0,
                rope_orig_max_seq=0, std=0.02, seed=1, threads=8, device=0, qk_norm=0, post_norms=0,
                sliding_window=0, layer_sliding=0, layer_local=0, rope_local_theta=0.0, rope_attn_factor=0.0,
                act=0, embed_scale=0.0, attn_softcap=0.0, final_softcap=0.0)
    base.update(kw)
    return base


CONFIGS = {
    "stories15m_q8": _spec(dim=288, n_layers=6, n_heads=6, n_kv_heads=6, hidden_dim=768, vocab=32000,
                           max_seq=256, seed=1),
    "qwen05b_mixed": _spec(dim=896, n_layers=24, n_heads=14, n_kv_heads=2, hidden_dim=4864, vocab=151936,
                           max_seq=1024, rope_theta=1e6, norm_eps=1e-6, wtype=ML_Q4_0,
                           q8_mask=Q8M_V | Q8M_O | Q8M_DOWN, shared=1, qkv_bias=1, scale_f16=1, seed=3),
    "llama1b_mixed": _spec(dim=2048, n_layers=16, n_heads=32, n_kv_heads=8, hidden_dim=8192, vocab=128256,
                           max_seq=4096, rope_theta=5e5, wtype=ML_Q4_0, q8_mask=Q8M_V | Q8M_O | Q8M_DOWN,
                           shared=1, scale_f16=1, rope_type=ML_ROPE_LLAMA3, rope_factor=32.0,
                           rope_low_freq_factor=1.0, rope_high_freq_factor=4.0, rope_orig_max_seq=8192, seed=4),
    "llama8b_q8": _spec(dim=4096, n_layers=32, n_heads=32, n_kv_heads=8, hidden_dim=14336, vocab=128256,
                        max_seq=4096, rope_theta=5e5, scale_f16=1, seed=5),
}


def _load(path):
    if not os.path.exists(path):
        raise RuntimeError("%s is not built: run __graft_entry__.build()" % path)
    return C.CDLL(path, mode=C.RTLD_GLOBAL)


class _Lib:
    """Only the declared functions of a library: calling an undeclared one
    through ctypes would pass 64-bit pointers as 32-bit ints."""

    def __init__(self, path):
        self._dll = _load(path)
        self._fns = {}

    def declare(self, name, res, args):
        f = getattr(self._dll, name)
        f.restype = res
        f.argtypes = args
        self._fns[name] = f

    def __getattr__(self, name):
        try:
            return self.__dict__["_fns"][name]
        except KeyError:
            raise AttributeError("%s is not declared in krafla.py" % name) from None

    def declared(self):
        return set(self._fns)


hip = _Lib(LIB_HIP)
host = _Lib(LIB_HOST)

_P = C.c_void_p
for name, res, args in [
    ("krh_init", C.c_int, []), ("krh_device_arch", C.c_char_p, []), ("krh_status", C.c_int, []),
    ("krh_device_cus", C.c_int, []), ("krh_ordered_sum_wave", None, [_P, _P, C.c_int, C.c_float]),
    ("krh_attention_noalloc", None, [_P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, _P]), ("krh_stream_read", None, [_P, _P, C.c_size_t, C.c_int]), ("krh_mfma_rate", None, [_P, C.c_int, C.c_int]),
    ("krh_last_error", C.c_char_p, []), ("krh_clear_error", None, []),
    ("krh_alloc", _P, [C.c_size_t]), ("krh_free", None, [_P]),
    ("krh_host_alloc", _P, [C.c_size_t]), ("krh_host_free", None, [_P]),
    ("krh_copy_h2d", C.c_int, [_P, _P, C.c_size_t]), ("krh_copy_d2h", C.c_int, [_P, _P, C.c_size_t]),
    ("krh_copy_d2d_async", None, [_P, _P, C.c_size_t]), ("krh_sync", C.c_int, []),
    ("krh_graph_begin", C.c_int, []), ("krh_graph_end", C.c_int, [C.POINTER(_P)]),
    ("krh_graph_launch", C.c_int, [_P]), ("krh_graph_free", None, [_P]),
    ("krh_timer_new", _P, []), ("krh_timer_mark", None, [_P, C.c_int]), ("krh_timer_ms", C.c_float, [_P]),
    ("krh_timer_free", None, [_P]),
    ("krh_embed", None, [_P, C.POINTER(KrhMat), _P, C.c_float]),
    ("krh_rmsnorm_q8", None, [_P, _P, _P, _P, _P, C.c_int, C.c_float, C.c_int]),
    ("krh_quantize_q8", None, [_P, _P, _P, C.c_int, C.c_int]),
    ("krh_matvec", None, [_P, C.POINTER(KrhMat), _P, _P, C.c_int]),
    ("krh_matvec_qkv", None, [_P, _P, _P, C.POINTER(KrhMat), C.POINTER(KrhMat), C.POINTER(KrhMat), _P, _P, _P,
                              _P, _P, _P, _P, C.c_int, _P]),
    ("krh_matvec_f", None, [_P, C.POINTER(KrhMat), _P, C.c_int]),
    ("krh_rmsnorm_matvec", None, [_P, C.POINTER(KrhMat), _P, _P, C.c_float, C.c_int]),
    ("krh_rmsnorm_matvec_qkv", None, [_P, _P, _P, C.POINTER(KrhMat), C.POINTER(KrhMat), C.POINTER(KrhMat), _P, _P,
                                      _P, _P, _P, C.c_float, _P, _P, C.c_int, _P]),
    ("krh_rmsnorm_matvec_swiglu", None, [_P, C.POINTER(KrhMat), C.POINTER(KrhMat), _P, _P, C.c_float]),
    ("krh_matvec_swiglu", None, [_P, C.POINTER(KrhMat), C.POINTER(KrhMat), _P, _P]),
    ("krh_attention", None, [_P, _P, _P, _P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                             _P]),
    ("krh_rmsnorm_matvec_qkv_f16", None, [_P, _P, _P, C.POINTER(KrhMat), C.POINTER(KrhMat), C.POINTER(KrhMat),
                                          _P, _P, _P, _P, _P, C.c_float, _P, _P, C.c_int, _P]),
    ("krh_rmsnorm_matvec_qkv_stage", None, [_P, _P, _P, C.POINTER(KrhMat), C.POINTER(KrhMat), C.POINTER(KrhMat),
                                            _P, _P, _P, _P, _P, C.c_float, _P, _P, C.c_int, _P]),
    ("krh_attention_kv", None, [_P, _P, _P, C.POINTER(MlKvLayer), C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                _P, C.c_int, C.c_int]),
    ("krh_attention_q8_store", None, [_P, _P, _P, C.POINTER(MlKvLayer), _P, _P, C.c_int, C.c_int, C.c_int, C.c_int,
                                      C.c_float, _P]),
    ("krh_store_kv", None, [C.c_int, _P, _P, _P, _P, _P, _P, C.c_int, C.c_int, _P, C.c_int]),
    ("krh_argmax", None, [_P, _P, C.c_int, _P, _P]),
    ("krh_sampler_new", C.c_int, [_P, C.c_int, _P]), ("krh_sampler_free", None, [_P]),
    ("krh_sampler_accept", None, [_P, _P, C.c_int]), ("krh_sample", None, [_P, _P, _P, C.c_int, _P, _P]),
    ("krh_sampler_rng", C.c_uint64, [_P]),
    ("krh_heads_norm_rope", None, [_P, _P, _P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_float, _P]),
    ("krh_store_rows_f32", None, [_P, _P, _P, _P, C.c_int, _P]),
    ("krh_softcap_att", None, [_P, C.c_int, C.c_int, C.c_int, _P, C.c_int, C.c_float]),
    ("krh_attention_kv_softcap", None, [_P, _P, _P, C.POINTER(MlKvLayer), C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, _P, C.c_int,
                                        C.c_int, C.c_float]),
    ("krh_tanhf_range", None, [_P, C.c_uint32, C.c_size_t]),
    ("krh_rmsnorm_q8_t", None, [_P, _P, C.c_int, _P, _P, _P, C.c_int, C.c_float, C.c_int]),
    ("krh_quantize_q8_t", None, [_P, _P, C.c_int, _P, C.c_int, C.c_int]),
    ("krh_matmul", None, [_P, C.c_int, C.POINTER(KrhMat), _P, _P, C.c_int, C.c_int, C.c_int]),
    ("krh_matmul_rows", None, [_P, C.c_int, C.POINTER(KrhMat), _P, _P, C.c_int, C.c_int, C.c_int]),
    ("krh_matmul_swiglu", None, [_P, _P, C.POINTER(KrhMat), C.POINTER(KrhMat), _P, _P, C.c_int, C.c_int]),
    ("krh_matmul_qkv", None, [_P, _P, _P, C.POINTER(KrhMat), C.POINTER(KrhMat), C.POINTER(KrhMat), _P, _P, _P,
                              _P, _P, C.c_int, C.c_int, _P, _P, C.c_int, C.c_int]),
    ("krh_matmul_qkv_stage", None, [_P, _P, _P, C.POINTER(KrhMat), C.POINTER(KrhMat), C.POINTER(KrhMat), _P, _P,
                                    _P, _P, _P, C.c_int, C.c_int, _P, _P, C.c_int, C.c_int]),
    ("krh_attention_batch", None, [_P, _P, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                   _P, C.c_int, C.c_int]),
    ("krh_set_attn_rb_min", None, [C.c_int]),
    ("krh_silu_quant", None, [_P, _P, C.c_int, _P, _P, C.c_int, C.c_int]),
    ("krh_embed_batch", None, [_P, C.POINTER(KrhMat), _P, C.c_int, C.c_float]),
    ("krh_take_token", None, [_P, _P, _P]), ("krh_advance", None, [_P]),
    ("krh_math_batch", None, [C.c_int, _P, _P, _P, C.c_size_t]), ("krh_h2f_batch", None, [_P, _P, C.c_size_t]),
    ("krh_block_dots", None, [_P, C.POINTER(KrhMat), _P]), ("krh_ordered_sum", None, [_P, _P, C.c_int, C.c_float]),
    ("krh_ordered_sum_1024", None, [_P, _P, C.c_int, C.c_float]),
    ("krh_ordered_sum_lean", None, [_P, _P, C.c_int, C.c_float]),
    ("krh_rmsnorm", None, [_P, _P, _P, C.c_int, C.c_float]), ("krh_add", None, [_P, _P, C.c_int]),
    ("krh_rope", None, [_P, _P, _P, _P, C.c_int, C.c_int, C.c_int]),
    ("krh_silu_mul", None, [_P, _P, C.c_int]), ("krh_gelu_mul", None, [_P, _P, C.c_int]),
    ("krh_softmax", None, [_P, C.c_int]),
    ("krh_dot_rows", None, [_P, _P, _P, C.c_size_t, C.c_int, C.c_int, C.c_float]),
    ("krh_axpy_rows", None, [_P, _P, _P, C.c_size_t, C.c_int, C.c_int]),
    ("krh_quantize_row", None, [_P, _P, _P, C.c_int]),
    ("krh_rmsnorm_rows", None, [_P, C.c_size_t, _P, C.c_size_t, _P, C.c_size_t, C.c_int, C.c_float, C.c_int]),
    ("krh_add_rows", None, [_P, C.c_size_t, _P, C.c_size_t, C.c_int, C.c_int]),
    ("krh_rope_rows", None, [_P, C.c_size_t, _P, C.c_size_t, _P, C.c_size_t, _P, C.c_size_t, C.c_int, C.c_int,
                             C.c_int, C.c_int]),
    ("krh_silu_mul_rows", None, [_P, C.c_size_t, _P, C.c_size_t, C.c_int, C.c_int]),
    ("krh_gelu_mul_rows", None, [_P, C.c_size_t, _P, C.c_size_t, C.c_int, C.c_int]),
    ("krh_quantize_row_rows", None, [_P, C.c_size_t, _P, C.c_size_t, _P, C.c_size_t, C.c_int, C.c_int]),
    ("krh_quantize_q8_rows", None, [_P, C.c_size_t, _P, C.c_size_t, _P, C.c_size_t, C.c_int, C.c_int]),
    ("krh_matvec_residual", None, [_P, _P, _P, _P, _P]),
    ("krh_matvec_multi", None, [_P, _P, C.c_int, _P, _P]),
    ("krh_matvec_swiglu_keep", None, [_P, _P, _P, _P, _P, _P]),
    ("krh_matvec_f_residual_keep", None, [_P, _P, _P, _P, _P, _P]),
    ("krh_rmsnorm_matvec_swiglu_keep", None, [_P, _P, _P, _P, _P, _P, C.c_float, _P, _P, _P]),
    ("krh_rmsnorm_matvec_qkv_keep", None, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, C.c_float, _P, _P, C.c_int,
                                           _P, _P, _P, _P]),
    ("krh_softcap_rows", None, [_P, C.c_size_t, C.c_int, C.c_int, C.c_float]),
    ("krh_set_int", None, [_P, C.c_int]),
    ("krh_gen_blocks", None, [_P, _P, C.c_uint64, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]),
]:
    hip.declare(name, res, args)

for name, res, args in [
    ("kr_status_str", C.c_char_p, [C.c_int]), ("kr_error", C.c_char_p, []),
    ("kr_model_load", C.c_int, [C.POINTER(_P), C.c_char_p]), ("kr_model_config", C.POINTER(MlConfig), [_P]),
    ("kr_model_tok_emb", C.POINTER(MlQTensor), [_P]), ("kr_model_layer", _P, [_P, C.c_int]), ("kr_model_wcls", C.POINTER(MlQTensor), [_P]),
    ("kr_model_upload", C.c_int, [_P]),
    ("kr_model_device_mat", C.POINTER(KrhMat), [_P, C.c_int, C.c_char_p]),
    ("kr_model_device_vec", _P, [_P, C.c_int, C.c_char_p]), ("kr_model_device_bytes", C.c_size_t, [_P]), ("kr_model_free", None, [_P]),
    ("kr_state_new", C.c_int, [C.POINTER(_P), _P, C.c_int]), ("kr_state_free", None, [_P]),
    ("kr_forward", C.c_int, [_P, C.c_int, C.c_int, _P]),
    ("kr_prefill", C.c_int, [_P, _P, C.c_int, C.c_int, _P]),
    ("kr_generate", C.c_int, [_P, _P, C.c_int, C.c_int, _P, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    ("kr_state_x_device", _P, [_P]), ("kr_state_buffer", _P, [_P, C.c_char_p]), ("kr_state_set_batch", None, [_P, C.c_int]),
    ("kr_state_set_sampler", C.c_int, [_P, _P]),
    ("kr_gen_mlb", C.c_int, [C.c_char_p, C.POINTER(GenSpec)]),
    ("kr_gen_matrix", None, [_P, _P, C.c_int, C.c_int, C.c_int, C.c_uint64, C.c_int]),
    ("kr_gen_normal", None, [_P, C.c_size_t, C.c_uint64]),
]:
    host.declare(name, res, args)


class KraflaError(RuntimeError):
    pass


def check(st, what=""):
    if st != ML_OK:
        detail = host.kr_error().decode(errors="replace") or hip.krh_last_error().decode(errors="replace")
        raise KraflaError("%s: %s (%s)" % (what, host.kr_status_str(st).decode(), detail))


def gen_mlb(path, threads=None, **spec):
    s = dict(spec)
    if threads is not None:
        s["threads"] = threads
    g = GenSpec(**s)
    check(host.kr_gen_mlb(path.encode(), C.byref(g)), "generate " + path)
    return path


def init_device():
    st = hip.krh_init()
    if st != ML_OK:
        raise KraflaError("no usable gfx950 device: " + hip.krh_last_error().decode(errors="replace"))


class SamplerOpts(C.Structure):
    """krh_sampler_opts: ml_sampler_opts (model/sampler.h:9-16), same layout"""
    _fields_ = [("temperature", C.c_float), ("topp", C.c_float), ("topk", C.c_int),
                ("repeat_penalty", C.c_float), ("repeat_last_n", C.c_int), ("seed", C.c_uint64)]


def sampler_opts(temperature=0.0, topp=0.9, topk=0, repeat_penalty=1.0, repeat_last_n=64, seed=1):
    """ml_run's defaults (app/ml_run.c:244-246)"""
    return SamplerOpts(temperature, topp, topk, repeat_penalty, repeat_last_n, seed)


class Sampler:
    """The device sampler (krh_sampler): ml_sample on device logits"""

    def __init__(self, vocab, opts):
        self.ptr = _P()
        check(hip.krh_sampler_new(C.byref(self.ptr), vocab, C.byref(opts)), "sampler")

    def accept(self, tokens_dev, n):
        """ml_sampler_accept of n ids at a device address"""
        hip.krh_sampler_accept(self.ptr, tokens_dev, n)

    def sample(self, tok_dev, logits_dev, n, pos_dev=None, log_dev=None):
        """the draw into *tok_dev (device addresses), then its accept"""
        hip.krh_sample(self.ptr, tok_dev, logits_dev, n, pos_dev, log_dev)

    @property
    def rng(self):
        return hip.krh_sampler_rng(self.ptr)

    def close(self):
        if self.ptr:
            hip.krh_sampler_free(self.ptr)
            self.ptr = _P()


class Model:
    def __init__(self, path):
        self.ptr = _P()
        check(host.kr_model_load(C.byref(self.ptr), path.encode()), "load " + path)
        self.cfg = host.kr_model_config(self.ptr).contents

    def upload(self):
        check(host.kr_model_upload(self.ptr), "upload")

    def close(self):
        if self.ptr:
            host.kr_model_free(self.ptr)
            self.ptr = _P()


class State:
    def __init__(self, model, kv_type=ML_F32):
        self.model = model
        self.ptr = _P()
        check(host.kr_state_new(C.byref(self.ptr), model.ptr, kv_type), "state")

    def forward(self, token, pos, out):
        """out: a float32 numpy array of vocab entries"""
        check(host.kr_forward(self.ptr, token, pos, out.ctypes.data), "forward")

    def set_batch(self, batch):
        host.kr_state_set_batch(self.ptr, batch)

    def set_sampler(self, opts):
        """the sampler generate() draws with (SamplerOpts), or None: greedy"""
        check(host.kr_state_set_sampler(self.ptr, C.byref(opts) if opts is not None else None), "sampler")

    def prefill(self, tokens, pos0, logits=None):
        import numpy as np
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        check(host.kr_prefill(self.ptr, t.ctypes.data, len(t), pos0,
                              logits.ctypes.data if logits is not None else None), "prefill")

    def generate(self, prompt, steps):
        import numpy as np
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max(steps, len(p)) + 2, dtype=np.int32)
        tp, td = C.c_double(), C.c_double()
        n = host.kr_generate(self.ptr, p.ctypes.data, len(p), steps, out.ctypes.data, C.byref(tp), C.byref(td))
        if n < 0:
            raise KraflaError("generate: " + (host.kr_error().decode() or hip.krh_last_error().decode()))
        return out[:n].copy(), tp.value, td.value

    def buffer(self, name, dtype, count):
        """a copy of an internal device buffer (tests)"""
        import numpy as np
        p = host.kr_state_buffer(self.ptr, name.encode())
        if not p:
            raise KeyError(name)
        out = np.empty(count, dtype=dtype)
        check(hip.krh_copy_d2h(out.ctypes.data, p, out.nbytes), "copy " + name)
        return out

    def close(self):
        if self.ptr:
            host.kr_state_free(self.ptr)
            self.ptr = _P()


class DevBuf:
    """A device allocation filled from / read into numpy arrays."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = hip.krh_alloc(max(self.nbytes, 1))
        if not self.ptr:
            raise KraflaError("device allocation of %d bytes failed" % nbytes)

    @classmethod
    def of(cls, arr):
        import numpy as np
        a = np.ascontiguousarray(arr)
        b = cls(a.nbytes)
        if a.nbytes:
            check(hip.krh_copy_h2d(b.ptr, a.ctypes.data, a.nbytes), "copy to device")
        return b

    def get(self, dtype, count):
        import numpy as np
        out = np.empty(count, dtype=dtype)
        if out.nbytes:
            check(hip.krh_copy_d2h(out.ctypes.data, self.ptr, out.nbytes), "copy to host")
        return out

    def free(self):
        if self.ptr:
            hip.krh_free(self.ptr)
            self.ptr = None
