"""The op-table binding's per-token op queue (isa-lm_amd/optable/kh_queue.h),
on the CPU: tests/csrc/queue_sim.c replays random per-token stages of row
ops, with planted cross-row hazards, through the queue and one call at a
time, and checks its overlap test against brute force. The queue's device
side runs in tests/test_gpu_optable.py (the reference's ml_run over the
binding, bit for bit against the scalar build)."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("qsim") / "queue_sim")
    subprocess.run(["gcc", "-O1", "-Wall", "-Werror", "-Wno-unused-parameter", "-I", os.path.join(ROOT, "include"),
                    "-I", os.path.join(ROOT, "isa-lm_amd", "optable"), os.path.join(HERE, "csrc", "queue_sim.c"),
                    "-o", exe, "-lm"], check=True)
    return exe


def run(exe, *args):
    return subprocess.run([exe] + [str(a) for a in args], capture_output=True, text=True, timeout=300)


def test_replay_matches_one_by_one(sim):
    r = run(sim, 3000)
    assert r.returncode == 0, r.stdout
    fields = r.stdout.split()
    calls, launches = int(fields[fields.index("calls") + 1]), int(fields[fields.index("launches") + 1])
    assert launches * 3 < calls, r.stdout   # the runs do batch


def test_wrong_overlap_test_is_caught(sim):
    """with "rows never overlap" in place of the overlap test the hazards
    show up as differing bytes"""
    r = run(sim, 3000, 1)
    assert r.returncode == 1 and "differs" in r.stdout, r.stdout


def test_overlap_test_against_brute_force(sim):
    r = run(sim, "meet", 1000000)
    assert r.returncode == 0, r.stdout


def test_fused_sequences_match_one_by_one(sim):
    """one token's decode sequences (model/transformer.c:270-293) launched as
    fused kernels leave the bytes of the calls one by one, with random
    aliasing among their buffers; every pattern fires"""
    r = run(sim, "fuse", 5000)
    assert r.returncode == 0, r.stdout


def test_fusion_without_alias_checks_is_caught(sim):
    r = run(sim, "fuse", 5000, 1)
    assert r.returncode == 1 and "differs" in r.stdout, r.stdout
