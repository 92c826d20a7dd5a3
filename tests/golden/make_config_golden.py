#!/usr/bin/env python3
"""Writes the golden fixtures of the full-size workloads from the reference's
scalar build (oracle/_ref/scalar/ml_run, compiled from the reference's own
sources by oracle/Makefile), in the build container.

For each workload (the Qwen2.5-0.5B, Llama-3.2-1B and Llama-3-8B shapes):
  1. the model is generated with the host generator (seeded; the device
     generator writes the same bytes) and its sha256 recorded;
  2. ml_run greedy-decodes the random prompt as the workload states
     (`ml_run M --tokens <prompt> -n <P-1+G> -T 0 -t N`, app/ml_run.c:369-404);
     its printed ids are kept (the prompt's ids after the first, then the G
     generated ones);
  3. ml_run --dump-logits runs the prompt followed by the generated ids
     (teacher-forced, app/ml_run.c:352-356): per position the sha256 of the
     float32 logits row (first 8 bytes), its argmax, maximum and float64 sum,
     and for three positions the top 64 logits with their ids.

THREADS=pthread does not change the scalar build's results
(tests/test_e2e.sh:175-181), so -t uses every core here.

Usage: python tests/golden/make_config_golden.py [workload ...]
Output: tests/golden/<workload>.npz (numpy, no pickles).
"""
import hashlib
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "isa-lm_amd"))
import krafla as K  # noqa: E402

ML_RUN = os.path.join(ROOT, "oracle", "_ref", "scalar", "ml_run")
OUT = os.path.dirname(os.path.abspath(__file__))

# workload: (prompt tokens P, generated tokens G, prompt seed)
WORKLOADS = {
    "qwen05b_mixed": (512, 256, 512),
    "llama1b_mixed": (4000, 96, 4000),
    "llama8b_q8": (2048, 256, 2048),
}


def log(msg):
    print("[golden] " + msg, file=sys.stderr, flush=True)


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
    """first 8 bytes of the sha256 of each row's float32 bytes, as uint64"""
    out = np.empty(logits.shape[0], dtype=np.uint64)
    for i in range(logits.shape[0]):
        out[i] = np.frombuffer(hashlib.sha256(logits[i].tobytes()).digest()[:8], dtype="<u8")[0]
    return out


def top_k(row, k=64):
    idx = np.argsort(-row.astype(np.float64), kind="stable")[:k].astype(np.int32)
    return idx, row[idx]


def make(name, workdir, threads):
    P, G, pseed = WORKLOADS[name]
    spec = dict(K.CONFIGS[name], threads=threads, device=0)
    vocab = spec["vocab"]
    path = os.path.join(workdir, name + ".mlb")
    t0 = time.time()
    K.gen_mlb(path, **spec)
    sha = file_sha256(path)
    log("%s: generated %.2f GB in %.1f s, sha256 %s" % (name, os.path.getsize(path) / 1e9, time.time() - t0, sha))
    prompt = np.random.default_rng(pseed).integers(1, vocab, P).astype(np.int32)
    toks = ",".join(str(int(t)) for t in prompt)

    n = P - 1 + G
    t0 = time.time()
    r = subprocess.run([ML_RUN, path, "--tokens", toks, "-n", str(n), "-T", "0", "-t", str(threads)],
                       capture_output=True, text=True, check=True)
    ids = np.array([int(v) for v in r.stdout.split()], dtype=np.int32)
    log("%s: greedy run %.0f s: %s" % (name, time.time() - t0, r.stderr.strip().replace("\n", " | ")))
    if ids.size != n or not np.array_equal(ids[:P - 1], prompt[1:]):
        raise SystemExit("%s: unexpected ml_run output (%d ids)" % (name, ids.size))

    forced = np.concatenate([prompt, ids[P - 1:-1]]).astype(np.int32)   # N = P + G - 1 positions
    dump = os.path.join(workdir, name + ".logits")
    t0 = time.time()
    r = subprocess.run([ML_RUN, path, "--tokens", ",".join(str(int(t)) for t in forced), "--dump-logits", dump,
                        "-t", str(threads)], capture_output=True, text=True, check=True)
    logits = np.fromfile(dump, dtype=np.float32).reshape(forced.size, vocab)
    os.remove(dump)
    log("%s: dump-logits run %.0f s" % (name, time.time() - t0))
    am = np.argmax(logits, axis=1).astype(np.int32)
    # the greedy ids are the teacher-forced argmaxes from the last prompt position on
    if not np.array_equal(am[P - 1:], ids[P - 1:]):
        raise SystemExit("%s: greedy ids differ from the dumped logits' argmax" % name)
    probe = np.array([0, P - 1, forced.size - 1], dtype=np.int32)
    tops = [top_k(logits[p]) for p in probe]
    np.savez_compressed(
        os.path.join(OUT, name + ".npz"),
        workload=np.array(name), mlb_sha256=np.array(sha), mlb_bytes=np.int64(os.path.getsize(path)),
        prompt=prompt, steps=np.int32(n), ids=ids, forced=forced,
        row_hash=row_hashes(logits), argmax=am, rowmax=logits.max(axis=1),
        rowsum=logits.astype(np.float64).sum(axis=1),
        probe_pos=probe, probe_ids=np.stack([t[0] for t in tops]), probe_vals=np.stack([t[1] for t in tops]),
        maker=np.array("oracle/_ref/scalar/ml_run -t %d (ISA=scalar THREADS=pthread)" % threads))
    os.remove(path)
    log("%s: wrote %s" % (name, os.path.join(OUT, name + ".npz")))


def main():
    names = sys.argv[1:] or list(WORKLOADS)
    workdir = os.environ.get("KR_GOLDEN_TMP", "/tmp/krgolden")
    os.makedirs(workdir, exist_ok=True)
    threads = int(os.environ.get("KR_GOLDEN_THREADS", str(os.cpu_count() or 8)))
    for name in names:
        make(name, workdir, threads)


if __name__ == "__main__":
    main()
