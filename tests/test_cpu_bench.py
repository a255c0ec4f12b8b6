"""bench.py's measured-traffic figures attach only to the configuration they were measured on."""

from __future__ import annotations

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_traffic_record_matches_only_its_configuration():
    layers = 32
    stack_bytes = layers * sum(bench._int8_bytes(r, c, 16) for _, r, c in bench.LAYER_SHAPES)
    measured = bench._traffic("int8_stack", stack_bytes, True)
    assert measured is not None and measured > stack_bytes
    assert bench._traffic("int8_stack", stack_bytes, False) is None      # measured with stochastic rounding
    one_layer = sum(bench._int8_bytes(r, c, 16) for _, r, c in bench.LAYER_SHAPES)
    assert bench._traffic("int8_stack", one_layer, True) is None         # another --layers
    K, N, r = 4096, 14336, 16
    routed = lambda t: 2 * (t * K + 2 * t * N + r * (K + N))  # noqa: E731
    assert bench._traffic("routed", routed(4096), False) is not None
    assert bench._traffic("routed", routed(1), False) is None            # another --tokens
    assert bench._traffic("no_such_workload", 1, False) is None
