"""The stream-K split (velokv_params.h sk_split / sk_begin / sk_worker_of,
sk_piece / sk_segment_workers), shared by the decode kernel and its merge,
compiled for the host with g++ and checked by brute force: contiguous non-empty
ranges within one unit of each other, the merge's unit -> worker map the exact
inverse of the kernel's worker -> range map, and, on random segment lists and
per-segment penalties, the kernel's walk over each worker's units runs every
block exactly once while the merge finds exactly the partials that cover each
split segment (slot 1 of its first worker, slot 0 of the rest, in order)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "velo-core_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not found")
def test_stream_k_split_is_consistent(tmp_path):
    exe = str(tmp_path / "sk_split_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", CSRC, os.path.join(HERE, "csrc", "sk_split_check.cpp"), "-o", exe],
                   check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr
