#!/usr/bin/env python3
"""Benchmark of the MI355X token loop on one GPU.

Workload (default): the Llama-3-8B-shaped model -- dim 4096, 32 layers,
32 query / 8 KV heads, head_dim 128, FFN 14336 SwiGLU, vocab 128256,
RoPE theta 5e5, every matrix Q8_0 in 32-blocks with f16 scales (8.53 GB),
random-init N(0, 0.02) from seed 5 -- run the way the reference's ml_run
runs a prompt (app/ml_run.c:369-404): a 2048-token random prompt
(ids uniform in [1, vocab)) of which 2047 tokens are prefilled, then
greedy decode, batch 1. A step is one decode token (one ml_forward plus the
greedy pick); `value` is decode tokens per second over --steps tokens at
positions 2047, 2048, ..., with the model and KV cache resident in HBM.

Also reported on the same line:
  prefill_tok_s   prompt tokens per second of the 2047-token prefill
  roofline        the dominant decode kernel as the decode step issues it:
                  the FFN rmsnorm + Q8_0 of x fused with the w1|w3 SwiGLU
                  matvec (54% of a layer's weight bytes); algorithmic bytes
                  per launch (weights + f16 scales of w1 and w3) over its
                  average launch duration, timed with HIP events on the
                  library stream around passes over all 32 layers (so the
                  weights come from HBM and not from the 256 MB Infinity
                  Cache); also against the measured plain HBM read rate (a
                  read-only streaming kernel over 4 GiB)
  roofline.traffic  HBM bytes per launch of that kernel, from the committed
                  rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE per
                  dispatch, each scaled by what the counter reads for k_add
                  of known traffic); the command that made it is
                  `bench.py --roofline-only`, which runs just the timed
                  SwiGLU launches and the calibration launches
  prefill_roofline  the dominant prefill kernel (the int8-MFMA matmul of w1
                  over the 2047 prompt tokens): int8 TOP/s against the
                  5.0 POP/s peak, against the exact-order VALU bound, and
                  against the measured int8 MFMA issue rate (a kernel of
                  back-to-back 32x32x32 MFMAs on register operands)
  matvec          the isolated Q4_0/Q8_0 matvec microbench (4096x4096 and
                  14336x4096, f16 scales, activation quantize_q8(N(0,1))):
                  GB/s over 1000 launches, cache-resident (one matrix) and
                  HBM-rotating (copies totalling more than 1 GB)
  cpu_baseline    the reference's best CPU build (avx512vnni, else avx2,
                  THREADS=pthread, built from its sources into oracle/_ref)
                  running ml_run on the same .mlb file and the same prompt
                  on this host's cores: the 2047-token prefill, then 32
                  greedy decode tokens at positions 2047..2078, the positions
                  the GPU decodes
  matvec_cpu_baseline  the reference's ml_bench kernel table (no model,
                  single-threaded) on one pinned core: its 4096x4096 matvec
                  rows in GB/s, beside the GPU matvec microbench
  reference_route (--reference-route) the reference's unchanged ml_run over
                  this backend's ISA=hip op table on the same model and
                  prompt: decode and prefill tok/s and whether its ids equal
                  the native loop's
"""
import argparse
import ctypes as C
import json
import os
import re
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "isa-lm_amd"))

METRIC = "decode tok/s (bs=1) + prefill tok/s on 1 MI355X; matvec HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
REF_DIR = os.path.join(ROOT, "oracle", "_ref")

WORKLOADS = {
    "llama8b_q8": ("llama3-8b-shape Q8_0 (f16 scales, 8.53 GB): 2048-token random prompt prefill, "
                   "then greedy decode, batch 1", 2048),
    "llama1b_mixed": ("llama3.2-1b-shape Q4_0 with Q8_0 v/o/down (f16 scales): 4000-token random prompt "
                      "prefill, then greedy decode over the 4096 KV cache, batch 1", 4000),
    "qwen05b_mixed": ("qwen2.5-0.5b-shape Q4_0 with Q8_0 v/o/down, tied, QKV bias: 512-token random prompt "
                      "prefill, then greedy decode, batch 1", 512),
    "stories15m_q8": ("llama2.c-15M-shape Q8_0 (f32 scales): 8-token random prompt, then greedy decode, "
                      "batch 1", 8),
}


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def scratch_dir(nbytes):
    for d in ("/dev/shm", tempfile.gettempdir()):
        try:
            if shutil.disk_usage(d).free > 2 * nbytes + (1 << 30):
                return tempfile.mkdtemp(prefix="krbench_", dir=d)
        except OSError:
            pass
    return tempfile.mkdtemp(prefix="krbench_")


def mat_bytes(W):
    n = W.rows * W.cols
    return (n if W.type == 1 else n // 2) + (n // 32) * (2 if W.d16 else 4)


def time_swiglu(K, model, state, reps):
    """average duration (ms) of the decode step's SwiGLU launch as the step
    issues it -- the FFN rmsnorm of the residual stream x, its Q8_0
    quantization and the w1|w3 matvec with SiLU(w1 x) * (w3 x), one fused
    launch (krh_rmsnorm_matvec_swiglu) -- over all layers, and its
    algorithmic bytes per launch: HIP events on the library stream around
    each pass over the layers (back-to-back launches, so the figure includes
    the gaps between them), divided by the launches"""
    cfg = model.cfg
    x = K.host.kr_state_buffer(state.ptr, b"x")
    hb = K.host.kr_state_buffer(state.ptr, b"hb")
    layers = [(K.host.kr_model_device_mat(model.ptr, l, b"w1"), K.host.kr_model_device_mat(model.ptr, l, b"w3"),
               K.host.kr_model_device_vec(model.ptr, l, b"ffn_norm")) for l in range(cfg.n_layers)]
    nbytes = mat_bytes(layers[0][0].contents) + mat_bytes(layers[0][1].contents)
    t = K.hip.krh_timer_new()
    total, n = 0.0, 0
    for _ in range(reps):
        K.hip.krh_timer_mark(t, 0)
        for w1, w3, nw in layers:
            K.hip.krh_rmsnorm_matvec_swiglu(hb, w1, w3, x, nw, cfg.norm_eps)
        K.hip.krh_timer_mark(t, 1)
        total += K.hip.krh_timer_ms(t)
        n += len(layers)
    K.hip.krh_timer_free(t)
    K.check(K.hip.krh_sync(), "swiglu timing")
    return total / n, nbytes


def hbm_read_peak(K, nbytes=4 << 30, reps=4):
    """the plain HBM read rate (GB/s): the best of a few launch shapes of a
    read-only streaming kernel (every 16-byte word of a 4 GiB buffer read
    once), HIP events around each launch"""
    buf, out = K.DevBuf(nbytes), K.DevBuf(4 * 65536)
    t = K.hip.krh_timer_new()
    best = 0.0
    cus = K.hip.krh_device_cus()
    for grid in (cus, 2 * cus, 8 * cus, 32 * cus, 64 * cus):
        K.hip.krh_stream_read(out.ptr, buf.ptr, nbytes, grid)
        for _ in range(reps):
            K.hip.krh_timer_mark(t, 0)
            K.hip.krh_stream_read(out.ptr, buf.ptr, nbytes, grid)
            K.hip.krh_timer_mark(t, 1)
            best = max(best, nbytes / (K.hip.krh_timer_ms(t) * 1e-3) / 1e9)
    K.check(K.hip.krh_sync(), "stream read")
    K.hip.krh_timer_free(t)
    buf.free()
    out.free()
    return round(best, 1)


def mfma_int8_rate(K, iters=4096, reps=3):
    """the achievable int8 MFMA rate (TOP/s): the best of a few grid sizes of
    a kernel issuing only 32x32x32 int8 MFMAs on register operands (four
    independent accumulators per wave), HIP events around each launch"""
    cus = K.hip.krh_device_cus()
    out = K.DevBuf(4 * 4 * 16 * cus)
    t = K.hip.krh_timer_new()
    best = 0.0
    for grid in (cus, 2 * cus, 4 * cus, 16 * cus // 4):
        K.hip.krh_mfma_rate(out.ptr, grid, iters)
        for _ in range(reps):
            K.hip.krh_timer_mark(t, 0)
            K.hip.krh_mfma_rate(out.ptr, grid, iters)
            K.hip.krh_timer_mark(t, 1)
            ops = 4.0 * grid * iters * 4 * 65536
            best = max(best, ops / (K.hip.krh_timer_ms(t) * 1e-3) / 1e12)
    K.check(K.hip.krh_sync(), "mfma rate")
    K.hip.krh_timer_free(t)
    out.free()
    return round(best, 1)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "swiglu_matvec_traffic.json")
CAL_N = 64 << 20   # k_add calibration: y += x over 64 Mi floats reads 512 MiB and writes 256 MiB


def calibration_adds(K, reps=3):
    """launches of k_add with known HBM traffic (y += x: 8 bytes read and 4
    written per element) for scaling the FETCH_SIZE / WRITE_SIZE counters"""
    y, x = K.DevBuf(4 * CAL_N), K.DevBuf(4 * CAL_N)
    for _ in range(reps):
        K.hip.krh_add(y.ptr, x.ptr, CAL_N)
    K.check(K.hip.krh_sync(), "calibration adds")
    y.free()
    x.free()


def committed_traffic():
    """HBM bytes per SwiGLU launch from the committed counter summary, or None;
    it was counted on the 8B shape's w1|w3 (its algorithmic_bytes), so other
    workloads report no traffic"""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def matvec_microbench(K, iters=1000):
    """GB/s of the plain matvec on the isolated shapes, resident and rotating:
    the 1000 launches captured as one graph and replayed (the host issues
    one graph launch, so the figure is the device's launches back to back,
    each graph kernel node's own dispatch cost included), and the same
    launches issued eagerly one by one from the host (eager_*: the host's
    issue rate included)"""
    out = []
    x = np.empty(4096, dtype=np.float32)
    K.host.kr_gen_normal(x.ctypes.data, 4096, 9)
    xb = K.DevBuf.of(x)
    xq, xdb = K.DevBuf(4096), K.DevBuf(4 * 128)
    K.hip.krh_quantize_q8(xq.ptr, xdb.ptr, xb.ptr, 4096, 1)
    t = K.hip.krh_timer_new()
    for typ, tname in ((2, "q4"), (1, "q8")):
        for rows in (4096, 14336):
            cols = 4096
            nq = rows * cols if typ == 1 else rows * cols // 2
            nd = rows * cols // 32
            nbytes = nq + 2 * nd
            q = np.empty(nq, dtype=np.uint8)
            d = np.empty(nd, dtype=np.uint16)
            K.host.kr_gen_matrix(q.ctypes.data, d.ctypes.data, rows, cols, typ, 11 + rows + typ, 16)
            copies = max(1, -(-(1 << 30) // nbytes))
            bufs = []
            for _ in range(copies):
                bufs.append((K.DevBuf.of(q), K.DevBuf.of(d)))
            yb = K.DevBuf(4 * rows)
            mats = [K.KrhMat(bq.ptr, bd.ptr, rows, cols, typ, 1) for bq, bd in bufs]
            res = {}
            for mode, seq in (("resident", [mats[0]] * iters), ("rotating", [mats[i % copies] for i in range(iters)])):
                for w in seq[:10]:
                    K.hip.krh_matvec(yb.ptr, C.byref(w), xq.ptr, xdb.ptr, 0)
                K.hip.krh_timer_mark(t, 0)
                for w in seq:
                    K.hip.krh_matvec(yb.ptr, C.byref(w), xq.ptr, xdb.ptr, 0)
                K.hip.krh_timer_mark(t, 1)
                ms = K.hip.krh_timer_ms(t)
                res["eager_" + mode] = round(nbytes * iters / (ms * 1e-3) / 1e9, 1)
                g = C.c_void_p()
                K.check(K.hip.krh_graph_begin(), "graph capture")
                for w in seq:
                    K.hip.krh_matvec(yb.ptr, C.byref(w), xq.ptr, xdb.ptr, 0)
                K.check(K.hip.krh_graph_end(C.byref(g)), "graph capture")
                K.check(K.hip.krh_graph_launch(g), "graph launch")   # warm: the graph's first replay uploads it
                K.hip.krh_timer_mark(t, 0)
                K.check(K.hip.krh_graph_launch(g), "graph launch")
                K.hip.krh_timer_mark(t, 1)
                ms = K.hip.krh_timer_ms(t)
                K.hip.krh_graph_free(g)
                res[mode] = round(nbytes * iters / (ms * 1e-3) / 1e9, 1)
                res[mode + "_us"] = round(ms * 1e3 / iters, 3)
            K.check(K.hip.krh_sync(), "matvec microbench")
            out.append({"shape": "%s %dx%d f16" % (tname, rows, cols), "bytes": nbytes,
                        "gbs_resident": res["resident"], "gbs_hbm_rotating": res["rotating"],
                        "us_per_launch_resident": res["resident_us"], "us_per_launch_rotating": res["rotating_us"],
                        "frac_hbm_rotating": round(res["rotating"] / HBM_PEAK_GBS, 3),
                        "eager_gbs_resident": res["eager_resident"], "eager_gbs_hbm_rotating": res["eager_rotating"]})
            for bq, bd in bufs:
                bq.free()
                bd.free()
            yb.free()
    K.hip.krh_timer_free(t)
    for b in (xb, xq, xdb):
        b.free()
    return out


def prefill_roofline(K, model, ntok, prefill_s, reps=2):
    """the dominant prefill kernel: the int8-MFMA matmul of w1 (hidden x dim)
    over ntok tokens, timed with HIP events over every layer's w1 on a random
    quantized activation batch; int8 ops = 2 * rows * cols * ntok per launch,
    against the 5.0 POP/s dense int8 peak and against the exact-order VALU
    bound (4 unfused VALU operations -- cvt, mul, mul, add -- per output and
    32-block, at 64 lanes x CUs x 2.4 GHz); plus the whole prefill's int8 ops
    over its wall time (attention, norms and launches included)"""
    cfg = model.cfg
    T = ntok
    ldx = (T + 127) // 128 * 128
    w1 = [K.host.kr_model_device_mat(model.ptr, l, b"w1") for l in range(cfg.n_layers)]
    rows, cols = w1[0].contents.rows, w1[0].contents.cols
    rng = np.random.default_rng(7)
    xq = K.DevBuf.of(rng.integers(-127, 128, ldx * cols).astype(np.int8))
    xd = K.DevBuf.of(np.abs(rng.normal(0, 0.01, (cols // 32) * ldx)).astype(np.float32))
    y = K.DevBuf(4 * T * rows)
    t = K.hip.krh_timer_new()
    K.hip.krh_matmul(y.ptr, rows, w1[0], xq.ptr, xd.ptr, ldx, T, 0)
    total, n = 0.0, 0
    for _ in range(reps):
        K.hip.krh_timer_mark(t, 0)
        for w in w1:
            K.hip.krh_matmul(y.ptr, rows, w, xq.ptr, xd.ptr, ldx, T, 0)
        K.hip.krh_timer_mark(t, 1)
        total += K.hip.krh_timer_ms(t)
        n += len(w1)
    K.check(K.hip.krh_sync(), "matmul timing")
    K.hip.krh_timer_free(t)
    for b in (xq, xd, y):
        b.free()
    us = total / n * 1e3
    mfma = mfma_int8_rate(K)
    ops = 2.0 * rows * cols * T
    tops = ops / (us * 1e-6) / 1e12
    valu_tops = 64 * K.hip.krh_device_cus() * 2.4e9 * (2 * 32 / 4) / 1e12   # int8 ops per exact-order VALU lane-op: 64 / 4
    layer_ops = 0
    for l in range(cfg.n_layers):
        for wn in (b"wq", b"wk", b"wv", b"wo", b"w1", b"w2", b"w3"):
            m = K.host.kr_model_device_mat(model.ptr, l, wn).contents
            layer_ops += 2.0 * m.rows * m.cols
    return {"bound": "valu (exact per-block rescale order)", "kernel": "k_matmul (w1, %dx%d, %d tokens)" % (rows, cols, T),
            "achieved": round(tops, 1), "peak": 5000.0, "unit": "TOP/s", "frac": round(tops / 5000.0, 4),
            "avg_launch_us": round(us, 1), "valu_bound": round(valu_tops, 1),
            "frac_of_valu_bound": round(tops / valu_tops, 4),
            "measured_mfma_int8_tops": mfma, "frac_of_measured_mfma": round(tops / mfma, 4) if mfma else None,
            "whole_prefill_int8_tops": round(layer_ops * T / prefill_s / 1e12, 1) if prefill_s else None}


def reference_route(path, prompt, decode, gpu_ids):
    """the reference's own ml_run, its model and app code unchanged, bound to
    this backend through the ISA=hip op table (oracle/_ref/hip/ml_run, built
    from the reference's sources by oracle/Makefile): the same model file and
    prompt, greedy, and whether its printed ids equal the native token loop's.
    Its prefill timer (app/ml_run.c:396-404) stops when the host has issued
    the prefill, before the device has run it, so the rates come from two
    runs' totals instead (positions / tok/s, app/ml_run.c:406-410): run A
    prefills and decodes one token, run B decodes `decode`; decode tok/s =
    (B positions - A positions) / (B time - A time), prefill tok/s =
    prefilled / (A time - one decode step)."""
    exe = os.path.join(REF_DIR, "hip", "ml_run")
    if not os.path.exists(exe):
        return {"value": None, "error": "oracle/_ref/hip/ml_run is not built"}

    def one(n):
        r = subprocess.run([exe, path, "--tokens", ",".join(str(int(t)) for t in prompt), "-n", str(n), "-T", "0"],
                           capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            raise RuntimeError("ml_run exited %d: %s" % (r.returncode, r.stderr[-300:]))
        qm = re.search(r"positions: (\d+), tok/s: ([\d.]+)", r.stderr)
        pm = re.search(r"prefill: (\d+) tokens in ([\d.]+) ms", r.stderr)
        pos = int(qm.group(1))
        return r.stdout, pos, pos / float(qm.group(2)), int(pm.group(1)) if pm else 0

    try:
        one(len(prompt))                                  # warm: page-in and first-launch costs
        _, pa, ta, P = one(len(prompt))
        out, pb, tb, _ = one(len(prompt) - 1 + decode)
    except RuntimeError as e:
        return {"value": None, "error": str(e)}
    ids = np.array([int(v) for v in out.split()], dtype=np.int32)
    step = (tb - ta) / (pb - pa)
    n = len(prompt) - 1 + decode
    k = min(len(ids), len(gpu_ids)) if gpu_ids is not None else 0
    return {"value": round((pb - pa) / (tb - ta), 3), "unit": "tok/s",
            "prefill_tok_s": round(P / (ta - step), 2) if P and ta > step else None,
            "ids_equal_native": bool(k == n and np.array_equal(ids[:k], gpu_ids[:k])) if gpu_ids is not None else None,
            "sample": "oracle/_ref/hip/ml_run (the reference's app/ml_run.c and model/transformer.c over the "
                      "ISA=hip op table), greedy: %d-token prompt (%d prefilled) run to %d and to %d positions; "
                      "decode tok/s = position difference / time difference, prefill tok/s = prefilled / "
                      "(first run's time - one decode step)" % (len(prompt), P, pa, pb)}


def cpu_matvec_baseline():
    """the reference's ml_bench kernel table (no model, app/ml_bench.c:37-61:
    single-threaded), pinned to one core, on its best CPU build: GB/s of the
    4096x4096 and 14336x4096-class matvec rows, weight and scale bytes as
    app/ml_bench.c:39 counts them"""
    for isa in ("avx512vnni", "avx2"):
        exe = os.path.join(REF_DIR, isa, "ml_bench")
        if not os.path.exists(exe):
            continue
        cmd = ([shutil.which("taskset"), "-c", str(min(os.sched_getaffinity(0)))] if shutil.which("taskset") else []) + [exe]
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
        if r.returncode == 3:
            continue
        if r.returncode != 0:
            return {"value": None, "error": "ml_bench %s exited %d" % (isa, r.returncode)}
        rows = []
        for line in r.stdout.splitlines():
            f = line.split()
            if len(f) >= 4 and f[0].startswith("matvec_") and f[1] in ("4096x4096",):
                rows.append({"op": f[0], "shape": f[1], "gbs": float(f[3])})
        return {"kind": "reference", "build": "ISA=%s" % isa, "cores": 1, "rows": rows,
                "sample": "ml_bench with no model (its kernel table), one pinned core"}
    return {"value": None, "error": "no reference CPU build in oracle/_ref"}


def cpu_baseline(path, prompt, decode, kv="f32", sample=None):
    """the reference's ml_run on the same model file, KV cache type and
    sampling options, on this host's cores"""
    cores = min(64, len(os.sched_getaffinity(0)))
    n = len(prompt) - 1 + decode
    for isa in ("avx512vnni", "avx2"):
        exe = os.path.join(REF_DIR, isa, "ml_run")
        if not os.path.exists(exe):
            continue
        cmd = [exe, path, "--tokens", ",".join(str(int(t)) for t in prompt), "-n", str(n), "-T", "0",
               "-t", str(cores), "--kv", kv]
        if sample:
            cmd += ["-T", repr(sample.temperature), "-p", repr(sample.topp), "--top-k", str(sample.topk),
                    "-s", str(sample.seed)]
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
        if r.returncode == 3:   # the reference's ISA guard: this CPU lacks the ISA
            continue
        if r.returncode != 0:
            return {"value": None, "error": "ml_run %s exited %d: %s" % (isa, r.returncode, r.stderr[-300:])}
        pm = re.search(r"prefill: (\d+) tokens in ([\d.]+) ms", r.stderr)
        qm = re.search(r"positions: (\d+), tok/s: ([\d.]+)", r.stderr)
        P, M = int(pm.group(1)), float(pm.group(2))
        pos, X = int(qm.group(1)), float(qm.group(2))
        dec = (pos - P) / (pos / X - M / 1000.0)
        cpu = ""
        try:
            with open("/proc/cpuinfo") as f:
                cpu = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
        except OSError:
            pass
        return {"value": round(dec, 3), "unit": "tok/s", "cores": cores, "kind": "reference",
                "build": "ISA=%s THREADS=pthread" % isa, "cpu": cpu,
                "sample": ("ml_run on the same .mlb: %d-token prompt (%d prefilled), %d %s decode tokens "
                           "at positions %d..%d; decode tok/s = (positions - prefilled) / (positions / tok/s - "
                           "prefill s)" % (len(prompt), P, pos - P, "sampled" if sample else "greedy",
                                           P, pos - 1)),
                "prefill_tok_s": round(P / (M / 1000.0), 2) if M > 0 else None}
    return {"value": None, "error": "no reference CPU build in oracle/_ref (build() needs the reference sources)"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode tokens")
    ap.add_argument("--warmup", type=int, default=16, help="untimed decode tokens before the timed run")
    ap.add_argument("--workload", default="llama8b_q8", choices=sorted(WORKLOADS))
    ap.add_argument("--prompt", type=int, default=None, help="prompt tokens (default: the workload's)")
    ap.add_argument("--kv", default="f32", choices=["f32", "f16", "q8"],
                    help="KV cache type (ml_run --kv): f32 is the headline configuration")
    ap.add_argument("--sample", default=None, metavar="T[,TOPP[,TOPK]]",
                    help="draw the decode tokens with the device sampler (ml_run -T, -p, --top-k; seed 1) "
                         "instead of the greedy pick")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-matvec", action="store_true")
    ap.add_argument("--reference-route", action="store_true",
                    help="also time the reference's unchanged ml_run over this backend's ISA=hip op table on the "
                         "same model and prompt")
    ap.add_argument("--route-only", action="store_true",
                    help="only the reference route on the generated model (for profiling it alone)")
    ap.add_argument("--roofline-reps", type=int, default=3)
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the timed SwiGLU launches and the k_add calibration launches (the command "
                         "the committed rocprofv3 counter summaries are made with)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the decode step would shard "
              "by output rows; see the design notes). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import krafla as K
    K.init_device()
    desc, P = WORKLOADS[args.workload]
    if args.prompt:
        P = args.prompt
    spec = dict(K.CONFIGS[args.workload], device=1)
    V = spec["vocab"]
    if P - 1 + max(args.steps, args.warmup) > spec["max_seq"]:
        sys.exit("prompt + steps exceed max_seq %d" % spec["max_seq"])
    est = 9 << 30 if args.workload == "llama8b_q8" else 2 << 30
    tmp = scratch_dir(est)
    path = os.path.join(tmp, args.workload + ".mlb")
    try:
        t0 = time.time()
        K.gen_mlb(path, **spec)
        log("generated %s (%.2f GB) in %.1f s" % (path, os.path.getsize(path) / 1e9, time.time() - t0))
        t0 = time.time()
        model = K.Model(path)
        kv_type = {"f32": K.ML_F32, "f16": K.ML_F16, "q8": K.ML_Q8_0}[args.kv]
        state = K.State(model, kv_type)
        dev_bytes = K.host.kr_model_device_bytes(model.ptr)
        log("uploaded %.2f GB to HBM in %.1f s" % (dev_bytes / 1e9, time.time() - t0))
        prompt = np.random.default_rng(2048).integers(1, V, P).astype(np.int32)
        if args.route_only:
            state.close()
            model.close()
            route = reference_route(path, prompt, args.steps, None)
            print(json.dumps({"workload": desc, "reference_route": route}), flush=True)
            return
        if args.roofline_only:
            ms, nbytes = time_swiglu(K, model, state, args.roofline_reps)
            calibration_adds(K)
            print(json.dumps({"swiglu_avg_launch_us": round(ms * 1e3, 2), "swiglu_bytes_per_launch": nbytes,
                              "swiglu_launches": args.roofline_reps * model.cfg.n_layers,
                              "calibration": {"kernel": "k_add", "n": CAL_N, "launches": 3,
                                              "read_bytes": 8 * CAL_N, "write_bytes": 4 * CAL_N}}), flush=True)
            state.close()
            model.close()
            return

        sample = None
        if args.sample:
            f = args.sample.split(",")
            sample = K.sampler_opts(temperature=float(f[0]), topp=float(f[1]) if len(f) > 1 else 0.9,
                                    topk=int(f[2]) if len(f) > 2 else 0)
            state.set_sampler(sample)   # a fresh sampler per run: the same draws
        ids_w, pre_w, _ = state.generate(prompt, P - 1 + args.warmup)
        if sample:
            state.set_sampler(sample)
        log("warmup: prefill %d tokens %.3f s, %d decode tokens" % (P - 1, pre_w, args.warmup))
        ids, pre_s, dec_s = state.generate(prompt, P - 1 + args.steps)
        n = min(len(ids_w), len(ids))
        deterministic = bool(np.array_equal(ids[:n], ids_w[:n]))
        tok_s = args.steps / dec_s
        prefill_tok_s = (P - 1) / pre_s if P > 1 else None
        log("timed: %d decode tokens in %.3f s (%.2f tok/s), prefill %.1f tok/s, ids deterministic: %s"
            % (args.steps, dec_s, tok_s, prefill_tok_s or 0.0, deterministic))

        ms, nbytes = time_swiglu(K, model, state, args.roofline_reps)
        gbs = nbytes / (ms * 1e-3) / 1e9
        log("rmsnorm + swiglu matvec: %.1f us per launch, %.1f GB/s" % (ms * 1e3, gbs))
        hbm = hbm_read_peak(K)
        log("plain HBM read rate: %.1f GB/s" % hbm)
        pre_rl = prefill_roofline(K, model, P - 1, pre_s)
        log("prefill matmul: %s" % json.dumps(pre_rl))
        cfg = model.cfg
        per_tok = 0
        for l in range(cfg.n_layers):
            for w in (b"wq", b"wk", b"wv", b"wo", b"w1", b"w2", b"w3"):
                per_tok += mat_bytes(K.host.kr_model_device_mat(model.ptr, l, w).contents)
        per_tok += mat_bytes(K.host.kr_model_device_mat(model.ptr, 0, b"wcls").contents)
        # KV cache: keys and values of positions 0..p read, row p written, at
        # the mean position of the timed tokens (elements of 4, 2 or 1 bytes;
        # the Q8 cache adds one float scale per KV head and row)
        p_mean = P - 1 + (args.steps - 1) / 2.0
        row = cfg.kv_dim * {"f32": 4, "f16": 2, "q8": 1}[args.kv] + (4 * cfg.n_kv_heads if args.kv == "q8" else 0)
        kv_tok = int(2 * cfg.n_layers * (p_mean + 2) * row)
        mv = None if args.no_matvec else matvec_microbench(K)
        mv_cpu = None
        if mv:
            for r in mv:
                log("matvec %s: %.1f GB/s resident, %.1f GB/s rotating" % (r["shape"], r["gbs_resident"],
                                                                           r["gbs_hbm_rotating"]))
            if not args.no_cpu_baseline:
                mv_cpu = cpu_matvec_baseline()
                log("matvec cpu baseline: %s" % json.dumps(mv_cpu))
        route = None
        if args.reference_route:
            t0 = time.time()
            route = reference_route(path, prompt, args.steps, ids)
            log("reference route (%.1f s): %s" % (time.time() - t0, json.dumps(route)))
        cpu = None
        if not args.no_cpu_baseline:
            t0 = time.time()
            cpu = cpu_baseline(path, prompt, min(32, args.steps), args.kv, sample)
            log("cpu baseline (%.1f s): %s" % (time.time() - t0, json.dumps(cpu)))
        state.close()
        model.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)

    traffic = committed_traffic()
    line = {
        "metric": METRIC, "value": round(tok_s, 3), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(1e3 * dec_s / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": desc, "prompt_tokens": P, "prefilled_tokens": P - 1, "decode_tokens": args.steps,
                   "first_decode_position": P - 1, "weight_bytes_per_token": per_tok,
                   "kv_cache": args.kv, "kv_bytes_per_token": kv_tok,
                   "sampler": ({"temperature": sample.temperature, "topp": sample.topp, "topk": sample.topk,
                                "seed": sample.seed} if sample else "greedy"),
                   "decode_roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / (per_tok + kv_tok), 1),
                   "parallelism": "single GPU"},
        "prefill_tok_s": round(prefill_tok_s, 2) if prefill_tok_s else None,
        "decode_frac_of_hbm_roofline": round(tok_s * (per_tok + kv_tok) / (HBM_PEAK_GBS * 1e9), 4),
        "deterministic_ids": deterministic,
        "roofline": {"bound": "hbm",
                     "kernel": "k_matvec<EPI_SWIGLU> with the rmsnorm prologue (krh_rmsnorm_matvec_swiglu: FFN "
                               "rmsnorm + Q8_0 of x, w1|w3 rows, SiLU(w1 x) * (w3 x)), as the decode step issues it",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic["bytes_per_launch"] if traffic and
                     traffic.get("algorithmic_bytes") == nbytes else None,
                     "bytes_per_launch": nbytes, "avg_launch_us": round(ms * 1e3, 2),
                     "measured_read_peak": hbm, "frac_of_measured_read_peak": round(gbs / hbm, 4)},
        "prefill_roofline": pre_rl,
        "matvec": mv,
        "matvec_cpu_baseline": mv_cpu,
        "cpu_baseline": cpu,
    }
    if route is not None:
        line["reference_route"] = route
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
