"""bench.py's block-timeline summary on hand-made stamps (CPU only): spans,
start spread, blocks per CU, in-flight counts and the per-bin byte rate."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_block_timeline_by_hand():
    # two blocks on one CU (XCC 0, CU field 1) over [0, 8) us, two on another
    # (XCC 1, CU field 2) over [4, 12) us; 100 ticks per us; windows 100 and 300
    hw = lambda cu: cu << 8
    st = np.array([[1000, 1800, hw(1), 0], [1000, 1800, hw(1), 0],
                   [1400, 2200, hw(2), 1], [1400, 2200, hw(2), 1]], np.uint64)
    r = bench.block_timeline(st, [100, 100, 300, 300])
    assert r["blocks"] == 4 and r["cus"] == 2 and r["blocks_per_cu"] == {"2": 2}
    assert r["span_us"] == 12.0 and r["last_start_us"] == 4.0
    assert r["block_us"]["50"] == 8.0 and r["cu_busy_us"]["100"] == 16.0
    assert r["mean_blocks_in_flight_per_cu"] == round(16 / 12, 2)
    assert r["blocks_in_flight_by_bin"] == [2.0, 4.0, 2.0]
    # a block reads window x 64 dims x (K, V) x 2 bytes over its 8 us
    low, high = 100 * 256 / 8 / 1e3, 300 * 256 / 8 / 1e3  # GB/s per block
    assert r["window_gbs_by_bin"] == [round(2 * low, 1), round(2 * low + 2 * high, 1),
                                      round(2 * high, 1)]
    assert r["ns_per_window_slot"]["10"] < r["ns_per_window_slot"]["90"]


def test_block_timeline_same_cu_id_on_two_xccs_counts_two_cus():
    st = np.array([[0, 100, 5 << 8, 0], [0, 100, 5 << 8, 3]], np.uint64)
    r = bench.block_timeline(st, [10, 20])
    assert r["cus"] == 2
    assert r["corr_block_us_window"] is None  # equal durations: no correlation to report
