"""Merge on reload (P/model_offloader.py:245-288 post-copy hooks, P/pinned_module.py:682-695) through
ReloadMergePipeline: every reload re-merges the pristine stored weights.  Each reloaded weight (per-row
INT8, per-row FP8, NVFP4 with one or two scale levels, plain or swizzled) equals the oracle's requant of
the GPU dense merge of the stored weight with seed derive_seed(path, merge_index); INT8 layers also
equal a grouped stack merge of copies of the stored weights with the same seeds."""

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


# ---- layers of mixed formats: per-row INT8, per-row FP8, two- and single-level NVFP4 ----
MIXED = (("q_proj", "int8", 64, 256), ("o_proj", "fp8", 48, 512), ("gate_proj", "nvfp4", 64, 512),
         ("up_proj", "nvfp4_1", 32, 256))


def _mixed_layers(n: int, rank: int = 16, swizzled: bool = False) -> list[list]:
    layers = []
    for li in range(n):
        layer = []
        for name, fmt, rows, cols in MIXED:
            w = normal_bf16((rows, cols), 0.02, 1000 * li + rows + cols)
            b, a = lora_factors(rows, cols, rank, 11 * li + cols)
            b, a = b.to(DEV), a.to(DEV)
            path, strength = f"layers.{li}.{name}.weight", 0.75 if li % 2 else 1.0
            if fmt == "int8":
                q, s = int8_initial(w)
                layer.append(R.HostInt8Target(path, q.pin_memory(), s.pin_memory(), b, a, strength))
            elif fmt == "fp8":
                s = (w.float().abs().amax(1, keepdim=True) / 448.0).clamp_min(2.0 ** -23)
                q = (w.float() / s).clamp(-448, 448).to(torch.float8_e4m3fn)
                layer.append(R.HostFloat8Target(path, q.pin_memory(), s.pin_memory(), b, a, strength))
            else:
                two = fmt == "nvfp4"
                q, sc, pts = O.nvfp4_requant(bf16_np(w), two_level=two, swizzled=swizzled)
                pt = None if pts is None else torch.from_numpy(pts.reshape(())).pin_memory()
                layer.append(R.HostNvfp4Target(path, torch.from_numpy(q).pin_memory(),
                                               torch.from_numpy(sc).view(torch.float8_e4m3fn).pin_memory(), pt,
                                               b, a, strength, swizzled))
        layers.append(layer)
    return layers


def _mixed_oracle(t, merge_index: int, stochastic: bool) -> list[np.ndarray]:  # noqa: ANN001
    """The oracle's requant of the GPU dense merge of one stored weight: [codes, scales(, global scale)]."""
    seed = derive_seed(t.path, merge_index) if stochastic else 0
    sr = O.SR_PHILOX8 if stochastic else O.SR_OFF
    lora = (t.b, t.a, t.strength)
    if isinstance(t, R.HostInt8Target):
        cols = t.qdata.shape[1]
        dense = K.dequantize_int8(t.qdata.to(DEV), t.scale.to(DEV), None, (1, cols), lora=lora)
        rq, rs, _ = O.int8_requant(bf16_np(dense), cols, sr_mode=sr, seed=seed)
        return [rq, rs]
    if isinstance(t, R.HostFloat8Target):
        cols = t.qdata.shape[1]
        dense = K.dequantize_float8(t.qdata.to(DEV), t.scale.to(DEV), (1, cols), lora=lora)
        rq, rs = O.fp8_requant(bf16_np(dense), cols, sr_mode=sr, seed=seed)
        return [rq, rs]
    pts = None if t.per_tensor_scale is None else t.per_tensor_scale.to(DEV)
    dense = K.dequantize_nvfp4(t.qdata.to(DEV), t.scale.to(DEV), pts, swizzled=t.is_swizzled_scales, lora=lora)
    rq, rs, rg = O.nvfp4_requant(bf16_np(dense), swizzled=t.is_swizzled_scales, two_level=pts is not None,
                                 sr_mode=sr, seed=seed)
    return [rq, rs] + ([rg] if rg is not None else [])


def _as_np(x: torch.Tensor) -> np.ndarray:
    x = x.detach().cpu().contiguous()
    if x.dtype in (torch.float8_e4m3fn, torch.float8_e5m2, torch.int8):
        x = x.view(torch.uint8) if x.dtype is not torch.int8 else x
    return x.numpy().reshape(-1)


@pytest.mark.parametrize("stochastic", [True, False])
@pytest.mark.parametrize("swizzled", [False, True])
def test_mixed_format_reloads_equal_the_oracle(stochastic: bool, swizzled: bool) -> None:
    layers = _mixed_layers(3, swizzled=swizzled)
    pipe = R.ReloadMergePipeline(layers, slots=2, stochastic=stochastic)
    for layer, mi in [(0, 0), (1, 0), (2, 0), (0, 1), (1, 4)]:
        got = pipe.reload(layer, mi)
        got.wait()
        for i, (w, t) in enumerate(zip(got.weights, layers[layer])):
            want = _mixed_oracle(t, mi, stochastic)
            have = [w.qdata, w.scale] + ([w.per_tensor_scale] if getattr(w, "per_tensor_scale", None) is not None
                                         else [])
            assert len(have) == len(want), f"layer {layer} target {i}"
            for k, (h, e) in enumerate(zip(have, want)):
                hv, ev = _as_np(h), np.asarray(e).reshape(-1)
                if hv.dtype != ev.dtype:
                    hv = hv.view(ev.dtype) if hv.itemsize == ev.itemsize else hv.astype(ev.dtype)
                m = mismatch_report(hv, ev, f"layer {layer} target {i} ({type(t).__name__}) part {k}", 64)
                assert not m, m
        pipe.release(got)
    pipe.synchronize()
    # the stored weights are untouched: a reload of layer 0 with index 0 repeats the first result
    again = pipe.reload(0, 0)
    again.wait()
    for w, t in zip(again.weights, layers[0]):
        want = _mixed_oracle(t, 0, stochastic)
        assert np.array_equal(_as_np(w.qdata).view(np.uint8), np.asarray(want[0]).reshape(-1).view(np.uint8))
