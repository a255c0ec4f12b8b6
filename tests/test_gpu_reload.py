"""Merge on reload (P/model_offloader.py:245-288 post-copy hooks) through
ReloadMergePipeline: every reload re-merges the pristine stored weights.  Each
reloaded weight equals the oracle's requant of the GPU dense merge of the
stored weight with seed derive_seed(path, merge_index), and a grouped stack
merge of copies of the stored weights with the same seeds."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import bf16_np, int8_initial, lora_factors, mismatch_report, normal_bf16

pytestmark = pytest.mark.gpu

R = pytest.importorskip("piper_offload_amd.reload")
K = pytest.importorskip("piper_offload_amd.kernels")
from piper_offload_amd import Int8Weight, derive_seed  # noqa: E402
from piper_offload_amd.stack import StackTarget, merge_int8_stack  # noqa: E402

DEV = "cuda"
SHAPES = (("q_proj", 64, 256), ("down_proj", 40, 384))


def _layers(n: int, rank: int = 16) -> list[list[R.HostInt8Target]]:
    layers = []
    for li in range(n):
        layer = []
        for name, rows, cols in SHAPES:
            q, s = int8_initial(normal_bf16((rows, cols), 0.02, 100 * li + rows))
            b, a = lora_factors(rows, cols, rank, 7 * li + cols)
            layer.append(R.HostInt8Target(f"layers.{li}.{name}.weight", q.pin_memory(), s.pin_memory(),
                                          b.to(DEV), a.to(DEV), 0.75 if li % 2 else 1.0))
        layers.append(layer)
    return layers


def _expected(layer: list[R.HostInt8Target], merge_index: int, stochastic: bool) -> list[Int8Weight]:
    ws = [Int8Weight(t.qdata.to(DEV), t.scale.to(DEV), (1, t.qdata.shape[1]), torch.bfloat16) for t in layer]
    merge_int8_stack([StackTarget(w, t.b, t.a, t.strength, derive_seed(t.path, merge_index))
                      for w, t in zip(ws, layer)], stochastic=stochastic)
    return ws


def _oracle(layer: list[R.HostInt8Target], merge_index: int, stochastic: bool) -> list[tuple]:
    """Per target: the oracle's requant of the GPU dense merge of the stored weight."""
    out = []
    for t in layer:
        cols = t.qdata.shape[1]
        dense = K.dequantize_int8(t.qdata.to(DEV), t.scale.to(DEV), None, (1, cols), lora=(t.b, t.a, t.strength))
        seed = derive_seed(t.path, merge_index)
        rq, rs, _ = O.int8_requant(bf16_np(dense), cols, sr_mode=O.SR_PHILOX8 if stochastic else O.SR_OFF,
                                   seed=seed if stochastic else 0)
        out.append((rq, rs))
    return out


def _check(got: R.Reloaded, want: list[Int8Weight], oracle: list[tuple] | None = None) -> None:
    got.wait()
    for g, w in zip(got.weights, want):
        assert torch.equal(g.qdata, w.qdata)
        assert torch.equal(g.scale, w.scale)
    for i, (g, (rq, rs)) in enumerate(zip(got.weights, oracle or [])):
        m = mismatch_report(g.qdata.cpu().numpy(), rq, f"target {i} codes vs oracle", 64)
        assert not m, m
        assert np.array_equal(g.scale.cpu().numpy().reshape(-1), rs), f"target {i} scales vs oracle"


@pytest.mark.parametrize("stochastic", [True, False])
def test_reloads_equal_stack_merges_of_the_stored_weights(stochastic: bool) -> None:
    layers = _layers(3)
    pipe = R.ReloadMergePipeline(layers, slots=2, stochastic=stochastic)
    order = [(0, 0), (1, 0), (2, 0), (0, 1), (1, 1), (0, 2)]
    for layer, mi in order:
        got = pipe.reload(layer, mi)
        _check(got, _expected(layers[layer], mi, stochastic), _oracle(layers[layer], mi, stochastic))
        pipe.release(got)
    # the stored weights are untouched
    again = pipe.reload(0, 1)
    _check(again, _expected(layers[0], 1, stochastic), _oracle(layers[0], 1, stochastic))


def test_two_reloads_in_flight_keep_their_own_slots() -> None:
    layers = _layers(2)
    pipe = R.ReloadMergePipeline(layers, slots=2)
    r0 = pipe.reload(0, 5)
    r1 = pipe.reload(1, 5)  # overlaps r0's merge on the copy stream
    assert r0.slot != r1.slot
    _check(r0, _expected(layers[0], 5, True))
    _check(r1, _expected(layers[1], 5, True))
    pipe.release(r0)
    pipe.release(r1)
    r2 = pipe.reload(1, 6)  # slot 0 again, after r0's release
    assert r2.slot == r0.slot
    _check(r2, _expected(layers[1], 6, True))


def test_merge_index_changes_the_stochastic_codes() -> None:
    layers = _layers(1)
    a = _expected(layers[0], 0, True)
    b = _expected(layers[0], 1, True)
    assert all(not torch.equal(x.qdata, y.qdata) for x, y in zip(a, b))
    # the scales come from the merged row maxima, which do not depend on the seed
    for x, y in zip(a, b):
        assert np.array_equal(x.scale.cpu().numpy(), y.scale.cpu().numpy())
