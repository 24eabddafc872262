"""The measurement's own arithmetic (CPU): the algorithmic bytes and flops
bench.py divides by, checked against the exact figures of BASELINE.json's five
configs (decode bytes = attended K + V + Q + O; prefill flops = 4 d x allowed
(query, key) pairs x heads), and the one-GPU contract of its command line."""
import os
import subprocess
import sys

import pytest

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("name,flops,bytes_,pairs", [
    # config 1: 2048 keys, all allowed
    ("decode_2k", None, 33_587_200, None),
    # config 2: the 1024-key window of a 32K cache (keys 31744..32767)
    ("decode_32k_window1024", None, 16_809_984, None),
    # config 2': the same cache, full causal (the 32K headline)
    ("decode_32k", None, 536_903_680, None),
    # config 3: 131072 keys, 16/2 heads, d 512
    ("decode_128k_d512", None, 1_073_807_360, None),
    # config 4a/4b: 4096 x 4096, causal with and without the 1024 window
    ("prefill_4k_window1024", 60_137_930_752, None, 3_670_528),
    ("prefill_4k", 137_472_507_904, None, 8_390_656),
    # config 5: 256 canvas queries over 2304 keys, non-causal (per step)
    ("canvas_256x2304", 9_663_676_416, 46_137_344, None),
    # the same prefill and canvas at the global-layer geometry (16/2, d 512)
    ("prefill_4k_d512", 274_945_015_808, None, 8_390_656),
    ("canvas_256x2304_d512", 19_327_352_832, None, None),
    # the output block of one token: W (2816 x 4096) + attended row + residual
    # + result, 2 x 4096 x 2816 flops
    ("output_decode", 23_068_672, 46_176_256, None),
    # the whole decode layer: the 32K attention plus that output block
    ("decode_32k_layer", 536_870_912 + 23_068_672, 536_903_680 + 46_176_256, None),
])
def test_algorithmic_work_matches_the_configs(name, flops, bytes_, pairs):
    f, b, p = bench.work(name)
    if flops is not None:
        assert f == flops
    if bytes_ is not None:
        assert b == bytes_
    if pairs is not None:
        assert p == pairs


def test_allowed_pairs_closed_forms():
    # causal n x n: n(n+1)/2; a window w: w(w+1)/2 + (n-w)w
    n, w = 4096, 1024
    assert bench.allowed_pairs(n, n, True, 0, 0) == n * (n + 1) // 2
    assert bench.allowed_pairs(n, n, True, w, 0) == w * (w + 1) // 2 + (n - w) * w
    assert bench.allowed_pairs(7, 30, False, 0, 0) == 7 * 30


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    assert res.stdout == ""
    assert "single MI355X" in res.stderr
