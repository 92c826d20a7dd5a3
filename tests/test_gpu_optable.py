"""The drop-in check of the ISA=hip op-table binding: the reference's own
app/ml_run.c and model/transformer.c, unchanged, built over
isa-lm_amd/optable and libkrafla_hip.so (oracle/Makefile `hip`), against the
reference's scalar build on the same .mlb files and token ids: the same
printed ids and the same --dump-logits bytes. Needs a gfx950 device."""
import os

import numpy as np
import pytest

import krafla as K
import oracle_lib as O

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not os.path.exists(os.path.join(O.REF_DIR, "hip", "ml_run")),
                                 reason="oracle/_ref/hip not built (needs the reference sources at build time)")]

MODELS = {
    "c1_q8": dict(K.CONFIGS["stories15m_q8"]),
    "qwen_like_q4mix": dict(K.CONFIGS["qwen05b_mixed"], dim=128, n_layers=3, n_heads=4, n_kv_heads=2,
                            hidden_dim=256, vocab=512, max_seq=160, std=0.1),
    "llama3_rope_gqa_q4": dict(K.CONFIGS["llama1b_mixed"], dim=256, n_layers=2, n_heads=8, n_kv_heads=2,
                               hidden_dim=512, vocab=1000, max_seq=200, std=0.1, rope_orig_max_seq=64),
    "q8_f16_untied": dict(K.CONFIGS["llama8b_q8"], dim=256, n_layers=2, n_heads=4, n_kv_heads=1, hidden_dim=384,
                          vocab=700, max_seq=160, std=0.1),
    # per-head q/k norms (heads_norm, model/transformer.c:246-248)
    "qk_norm_q4mix": dict(K.CONFIGS["qwen05b_mixed"], dim=128, n_layers=2, n_heads=4, n_kv_heads=2, hidden_dim=256,
                          vocab=512, max_seq=400, std=0.1, qk_norm=1, qkv_bias=0),
    # post-norms, GELU, sliding-window layers with the local RoPE base
    "post_norm_gelu_window": dict(K.CONFIGS["stories15m_q8"], dim=128, n_layers=3, n_heads=4, n_kv_heads=1,
                                  hidden_dim=256, vocab=600, max_seq=400, std=0.1, qk_norm=1, post_norms=1, act=1,
                                  sliding_window=40, layer_sliding=0b101, layer_local=0b101, rope_local_theta=1e4,
                                  rope_theta=1e6),
    # the embedding's scale (applied on the device by ml_dequant_row) and
    # soft-capped scores and logits
    "softcap_embed_scale": dict(K.CONFIGS["stories15m_q8"], dim=128, n_layers=2, n_heads=4, n_kv_heads=2,
                                hidden_dim=256, vocab=600, max_seq=400, std=0.1, post_norms=1, act=1,
                                embed_scale=11.3137, attn_softcap=50.0, final_softcap=30.0, sliding_window=32,
                                layer_sliding=0b01),
}


def model(name, workdir):
    path = os.path.join(workdir, "ot_" + name + ".mlb")
    if not os.path.exists(path):
        K.gen_mlb(path, **MODELS[name])
    return path


@pytest.mark.parametrize("name", sorted(MODELS))
def test_ml_run_greedy_ids(name, workdir):
    path = model(name, workdir)
    V = MODELS[name]["vocab"]
    prompt = [int(t) for t in np.random.default_rng(3).integers(1, V, 8)]
    steps = min(MODELS[name]["max_seq"], 8 + 128)
    want, _ = O.ref_ml_run(path, prompt, steps)
    got, err = O.ref_ml_run(path, prompt, steps, isa="hip")
    assert "isa: hip" in err
    assert np.array_equal(got, want)


@pytest.mark.parametrize("batch", [None, 1])
@pytest.mark.parametrize("name", sorted(MODELS))
def test_ml_run_dump_logits(name, batch, workdir):
    path = model(name, workdir)
    V = MODELS[name]["vocab"]
    toks = [int(t) for t in np.random.default_rng(4).integers(1, V, 20)]
    a, b = path + ".scalar.logits", path + ".hip.logits"
    O.ref_ml_run(path, toks, len(toks), dump=a)
    O.ref_ml_run(path, toks, len(toks), dump=b, isa="hip", extra=["--batch", str(batch)] if batch else [])
    x, y = np.fromfile(a, dtype=np.uint8), np.fromfile(b, dtype=np.uint8)
    assert x.size == len(toks) * V * 4 and np.array_equal(x, y)


def test_ml_bench_kernel_table():
    """ml_bench (no model) runs its kernel table on the hip kernels, staged
    from host buffers (the build with the reference's default 128-token
    batches, app/ml_bench.c:53-54)"""
    import subprocess
    r = subprocess.run([os.path.join(O.REF_DIR, "hip128", "ml_bench")], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr
    assert "ISA: hip" in r.stdout and "matvec_q8 -> ml_k_matvec_q8_hip" in r.stdout


@pytest.mark.parametrize("build", ["hip", "hip128"])
@pytest.mark.parametrize("kv", ["f32", "q8", "f16"])
def test_ml_bench_model_mode(kv, build, workdir):
    """ml_bench with a model (app/ml_bench.c:105-131): ml_prefill of 64
    tokens, then 64 ml_forward steps with an inline argmax, through the op
    table; it prints only rates, so the check is that the run completes on
    the device and reports both"""
    import re
    import subprocess
    path = model("qwen_like_q4mix", workdir)
    r = subprocess.run([os.path.join(O.REF_DIR, build, "ml_bench"), path, "-n", "64", "--kv", kv],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr
    m = re.search(r"model .*: prefill ([\d.]+) tok/s, decode ([\d.]+) tok/s \(64 tokens each", r.stdout)
    assert m and float(m.group(1)) > 0 and float(m.group(2)) > 0, r.stdout
    assert "error" not in r.stderr


@pytest.mark.parametrize("build", ["hip", "hip128"])
@pytest.mark.parametrize("name", ["c1_q8", "qwen_like_q4mix", "llama3_rope_gqa_q4", "softcap_embed_scale"])
def test_ml_run_imatrix(name, build, workdir):
    """--imatrix (app/ml_run.c:104-170, model/transformer.c:250-255): the
    importance file written over the op table equals the reference's byte
    for byte (its float64 sums of every matrix input's squares, per channel,
    through the batched prefill and the per-token decode), and a second run
    adds to it as the reference's does"""
    path = model(name, workdir)
    V = MODELS[name]["vocab"]
    prompt = [int(t) for t in np.random.default_rng(6).integers(1, V, 24)]
    a, b = path + ".scalar.imat", path + "." + build + ".imat"
    for f in (a, b):
        if os.path.exists(f):
            os.remove(f)
    for rep in range(2):
        want, _ = O.ref_ml_run(path, prompt, 48, extra=["--imatrix", a])
        got, err = O.ref_ml_run(path, prompt, 48, isa=build, extra=["--imatrix", b])
        assert np.array_equal(got, want)
        x, y = np.fromfile(a, dtype=np.uint8), np.fromfile(b, dtype=np.uint8)
        assert x.size > 40 and np.array_equal(x, y), rep


@pytest.mark.parametrize("batch", [None, 1])
@pytest.mark.parametrize("name", ["c1_q8", "llama3_rope_gqa_q4", "qwen_like_q4mix"])
def test_ml_run_kv_q8(name, batch, workdir):
    """--kv q8 (app/ml_run.c:277-281): store_kv quantizes through
    ml_quantize_row on the device, attention reads the Q8 rows; the same
    --dump-logits bytes and ids as the scalar build"""
    path = model(name, workdir)
    V = MODELS[name]["vocab"]
    toks = [int(t) for t in np.random.default_rng(4).integers(1, V, 20)]
    a, b = path + ".scalar.q8.logits", path + ".hip.q8.logits"
    O.ref_ml_run(path, toks, len(toks), dump=a, extra=["--kv", "q8"])
    O.ref_ml_run(path, toks, len(toks), dump=b, isa="hip",
                 extra=["--kv", "q8"] + (["--batch", str(batch)] if batch else []))
    x, y = np.fromfile(a, dtype=np.uint8), np.fromfile(b, dtype=np.uint8)
    assert x.size == len(toks) * V * 4 and np.array_equal(x, y)
    steps = min(MODELS[name]["max_seq"], 8 + 64)
    want, _ = O.ref_ml_run(path, toks[:8], steps, extra=["--kv", "q8"])
    got, _ = O.ref_ml_run(path, toks[:8], steps, isa="hip", extra=["--kv", "q8"])
    assert np.array_equal(got, want)


@pytest.mark.parametrize("build", ["hip", "hip128"])
@pytest.mark.parametrize("batch", [None, 1])
@pytest.mark.parametrize("name", ["c1_q8", "llama3_rope_gqa_q4", "qwen_like_q4mix", "qk_norm_q4mix",
                                  "post_norm_gelu_window"])
def test_ml_run_kv_f16(name, batch, build, workdir):
    """--kv f16 (app/ml_run.c:277-281): store_kv's host loop converts K and V
    to halves (model/transformer.c:195-197) from staging rows that live on
    the device; the binding converts them on the device before attention
    reads the cache. The same --dump-logits bytes and greedy ids as the
    scalar build's --kv f16, per token (--batch 1) and batched (one step, or
    the 128-token steps of hip128 over a 150-token prompt)"""
    path = model(name, workdir)
    V, S = MODELS[name]["vocab"], MODELS[name]["max_seq"]
    n = min(150, S - 40)
    toks = [int(t) for t in np.random.default_rng(8).integers(1, V, n)]
    a, b = path + ".scalar.f16.logits", path + "." + build + ".f16.logits"
    ext = ["--kv", "f16"] + (["--batch", str(batch)] if batch else [])
    O.ref_ml_run(path, toks, n, dump=a, extra=["--kv", "f16"])
    O.ref_ml_run(path, toks, n, dump=b, isa=build, extra=ext)
    x, y = np.fromfile(a, dtype=np.uint8), np.fromfile(b, dtype=np.uint8)
    assert x.size == n * V * 4 and np.array_equal(x, y)
    steps = min(S, 8 + 64)
    want, _ = O.ref_ml_run(path, toks[:8], steps, extra=["--kv", "f16"])
    got, _ = O.ref_ml_run(path, toks[:8], steps, isa=build, extra=ext)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("build", ["hip", "hip128"])
@pytest.mark.parametrize("name", ["qk_norm_q4mix", "post_norm_gelu_window", "softcap_embed_scale",
                                  "llama3_rope_gqa_q4", "c1_q8"])
def test_ml_run_long_prompt(name, build, workdir):
    """A prompt of up to 300 tokens: in one batched prefill step (hip:
    ML_BATCH_MAX 2048), or over several of the reference's default 128-token
    steps (hip128, model/transformer.h:48); the binding replays each step's
    per-token op loops as row-batched launches; the --dump-logits bytes and
    the greedy ids that follow match the scalar build's"""
    path = model(name, workdir)
    V, S = MODELS[name]["vocab"], MODELS[name]["max_seq"]
    n = min(300, S - 40)
    toks = [int(t) for t in np.random.default_rng(5).integers(1, V, n)]
    a, b = path + ".scalar.long.logits", path + "." + build + ".long.logits"
    O.ref_ml_run(path, toks, n, dump=a)
    O.ref_ml_run(path, toks, n, dump=b, isa=build)
    x, y = np.fromfile(a, dtype=np.uint8), np.fromfile(b, dtype=np.uint8)
    assert x.size == n * V * 4 and np.array_equal(x, y)
    want, _ = O.ref_ml_run(path, toks, n + 32)
    got, _ = O.ref_ml_run(path, toks, n + 32, isa=build)
    assert np.array_equal(got, want)


def test_ml_run_batch_option(workdir):
    """--batch up to the build's ML_BATCH_MAX (app/ml_run.c:274): the 2048
    build takes --batch 2048 and 200, the 128 build refuses 129"""
    import subprocess
    path = model("qwen_like_q4mix", workdir)
    toks = [int(t) for t in np.random.default_rng(6).integers(1, 512, 150)]
    want, _ = O.ref_ml_run(path, toks, 158)
    for b in ("2048", "200", "7"):
        got, _ = O.ref_ml_run(path, toks, 158, isa="hip", extra=["--batch", b])
        assert np.array_equal(got, want), b
    r = subprocess.run([os.path.join(O.REF_DIR, "hip128", "ml_run"), path, "--tokens", "1,2", "-n", "3",
                        "--batch", "129"], capture_output=True, text=True, timeout=300)
    assert r.returncode != 0 and "--batch" in r.stderr
