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
    # the global-layer decode at 32K keys: 2 x 32768 x 2 x 512 x 4 + 2 x 16 x 512 x 4
    ("decode_32k_d512", None, 268_500_992, None),
    # the reference's probe shapes (int8/tests.rs:770-809), 8 queries over
    # every key: K + V = 2 x 1279 x 8 x 256 x 4, Q + O = 2 x 8 x 16 x 256 x 4
    ("probe_sliding_q8", 4 * 256 * 8 * 1279 * 16, 20_955_136 + 262_144, 8 * 1279),
    # K + V = 2 x 3194 x 2 x 512 x 4, Q + O = 2 x 8 x 16 x 512 x 4
    ("probe_global_q8", 4 * 512 * 8 * 3194 * 16, 26_165_248 + 524_288, 8 * 3194),
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


def test_probe_rate_is_the_references_gmacs():
    # int8/tests.rs:800-806: macs = 2 nq qheads nkeys dim per call
    assert bench.reference_gmacs("probe_sliding_q8", 1.0) * 1e9 == 2 * 8 * 16 * 1279 * 256
    assert bench.reference_gmacs("probe_global_q8", 0.5) * 1e9 == 4 * 8 * 16 * 3194 * 512


def test_every_baseline_config_has_a_cpu_leg():
    for name in ("decode_2k", "decode_32k_window1024", "decode_32k", "decode_128k_d512",
                 "prefill_4k_window1024", "prefill_4k", "canvas_256x2304"):
        assert name in bench.CPU_LEGS
        if bench.WORKLOADS[name][8] != "decode":
            assert name in bench.ROW_SAMPLE
