"""bench.py's CPU-baseline leg on a tiny generated model (CPU only): the
reference's ml_run build in oracle/_ref runs it, and the result record is
formed from its stderr (app/ml_run.c:406-410)."""
import importlib.util
import os
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "isa-lm_amd"))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("sample", [None, "0.8,0.9"])
def test_cpu_baseline_record(sample):
    bench = _bench()
    if not any(os.path.exists(os.path.join(bench.REF_DIR, isa, "ml_run")) for isa in ("avx512vnni", "avx2")):
        pytest.skip("no reference CPU build in oracle/_ref")
    import krafla as K
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "tiny.mlb")
        K.gen_mlb(path, **dict(K.CONFIGS["stories15m_q8"], n_layers=2, seed=3))
        smp = K.sampler_opts(temperature=0.8, topp=0.9, topk=0) if sample else None
        rec = bench.cpu_baseline(path, [1, 5, 9, 13, 17, 21, 25, 29], 16, "f32", smp)
    assert rec.get("value") is not None and rec["value"] > 0, rec
    assert rec["unit"] == "tok/s" and rec["kind"] == "reference" and rec["cores"] >= 1
    assert "8-token prompt (7 prefilled), 16 %s decode tokens at positions 7..22" % (
        "sampled" if sample else "greedy") in rec["sample"]
