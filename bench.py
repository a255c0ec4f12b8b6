#!/usr/bin/env python3
"""LoRA-merge throughput on one MI355X.

Default workload (BASELINE.json metric "LoRA-merge GB/s & % of HBM peak; ms to
merge 8B-shaped INT8 stack", config 5): the 224 projection weights of an
8B-shaped model (32 layers x q/o [4096,4096], k/v [1024,4096], gate/up
[14336,4096], down [4096,14336]) stored as per-row symmetric INT8 with fp32
scales, a rank-16 bf16 LoRA on every projection (A ~ N(0, 1/16),
B ~ N(0, 0.01), strength 1.0), stochastic requant with one Philox seed per
target and merge index, derive_seed(param_path, step).  A step merges the
whole stack once, in place, through the grouped HIP kernel.

``value`` is algorithmic GB/s: per target 2*M*N (codes in + out) + 8*M
(fp32 scales in + out) + 2*r*(M+N) (bf16 factors), over the step time.  The
``roofline`` block uses the dominant kernel's own HIP-event time, taken over
a second run of K steps (per-launch events would slow the first); the
``cpu_baseline`` block times the reference's portable merge (dequantize,
addmm_, requantize) in torch CPU ops on the host cores, on a bounded sample of
the same workload.

    python bench.py [--steps K] [--warmup W]
                    [--workload int8_stack|nvfp4_stack|int8|fp8|q8_0|nvfp4|mxfp4|gguf|reload|h2d|copy]
                    [--rounding stochastic|nearest] [--gguf-type Q4_K] [--cpu-seconds S]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "piper-offload_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth
METRIC = "LoRA-merge GB/s & % of HBM peak; ms to merge 8B-shaped INT8 stack"

LAYER_SHAPES = (
    ("self_attn.q_proj", 4096, 4096),
    ("self_attn.k_proj", 1024, 4096),
    ("self_attn.v_proj", 1024, 4096),
    ("self_attn.o_proj", 4096, 4096),
    ("mlp.gate_proj", 14336, 4096),
    ("mlp.up_proj", 14336, 4096),
    ("mlp.down_proj", 4096, 14336),
)


GGUF_TYPES = {"F32": 0, "F16": 1, "BF16": 30, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q2_K": 10,
              "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_NL": 20, "IQ4_XS": 23}
# byte offsets of the fp16 fields (d, dmin / m) of each GGUF block struct
GGUF_F16_FIELDS = {2: (0,), 3: (0, 2), 6: (0,), 7: (0, 2), 8: (0,), 20: (0,), 10: (80, 82), 11: (108,),
                   12: (0, 2), 13: (0, 2), 14: (208,), 23: (0,)}


def _gguf_bytes(qtype: int, rows: int, cols: int, seed: int):  # noqa: ANN202
    """Random GGUF blocks of one type (finite fp16 scale fields) as a numpy uint8 [rows, row_bytes]."""
    import numpy as np

    from piper_offload_amd.gguf_dequant import GGML_QUANT_SIZES

    bs, ts = GGML_QUANT_SIZES[qtype]
    rng = np.random.default_rng(seed)
    nblk = rows * cols // bs
    if qtype in (0, 1, 30):
        vals = (rng.standard_normal(rows * cols, dtype=np.float32) * 0.02)
        raw = vals.view(np.uint8) if qtype == 0 else (
            vals.astype(np.float16).view(np.uint8) if qtype == 1 else (vals.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8))
        return np.ascontiguousarray(raw).reshape(rows, -1)
    raw = rng.integers(0, 256, (nblk, ts), dtype=np.uint8)
    for off in GGUF_F16_FIELDS[qtype]:
        raw[:, off:off + 2] = (rng.uniform(1e-4, 1e-3, nblk).astype(np.float16)).view(np.uint8).reshape(nblk, 2)
    return raw.reshape(rows, -1)


def _parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", default="int8_stack",
                   choices=["int8_stack", "nvfp4_stack", "int8", "fp8", "q8_0", "nvfp4", "mxfp4", "gguf", "reload", "h2d",
                            "api", "routed", "copy"])
    p.add_argument("--gguf-type", default="Q4_K", choices=sorted(GGUF_TYPES),
                   help="GGUF type of --workload gguf (dequantize to bf16)")
    p.add_argument("--rounding", default="stochastic", choices=["stochastic", "nearest"])
    p.add_argument("--layers", type=int, default=32)
    p.add_argument("--tokens", type=int, default=4096, help="tokens of --workload routed")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of the CPU-oracle baseline (0: skip)")
    return p.parse_args()


# ---------------------------------------------------------------------------
# synthetic workloads
# ---------------------------------------------------------------------------
def _gen(seed: int):  # noqa: ANN202
    import torch

    return torch.Generator(device="cuda").manual_seed(seed % (1 << 63))


def _normal(shape, std, seed, dtype=None):  # noqa: ANN001, ANN202
    import torch

    t = torch.randn(shape, generator=_gen(seed), device="cuda", dtype=torch.float32).mul_(std)
    return t.to(dtype or torch.bfloat16)


def _int8_weight(path: str, rows: int, cols: int):  # noqa: ANN202
    import torch

    from piper_offload_amd import Int8Weight, derive_seed

    w = _normal((rows, cols), 0.02, derive_seed(path, 0)).float()
    scale = (w.abs().amax(dim=1, keepdim=True) / 127.0).clamp_min(torch.finfo(torch.float32).eps)
    q = torch.round(w / scale).clamp_(-128, 127).to(torch.int8)
    del w
    return Int8Weight(q, scale, (1, cols), torch.bfloat16)


def _nvfp4_weight(path: str, rows: int, cols: int):  # noqa: ANN202
    from piper_offload_amd import NVFP4Weight, derive_seed
    from piper_offload_amd.kernels import requantize_nvfp4

    w = _normal((rows, cols), 0.02, derive_seed(path, 0))
    q, s, pts = requantize_nvfp4(w, two_level=True, swizzled=False)
    del w
    return NVFP4Weight(q, s, pts.reshape(()), 16)


def _factors(path: str, rows: int, cols: int, rank: int):  # noqa: ANN202
    from piper_offload_amd import derive_seed

    a = _normal((rank, cols), 1.0 / rank, derive_seed(path, 1))
    b = _normal((rows, rank), 0.01, derive_seed(path, 2))
    return b, a


def _int8_bytes(rows: int, cols: int, rank: int) -> int:
    return 2 * rows * cols + 8 * rows + 2 * rank * (rows + cols)


def _nvfp4_bytes(rows: int, cols: int, rank: int) -> int:
    return 2 * (rows * cols // 2 + rows * cols // 16) + 8 + 2 * rank * (rows + cols)


class Workload:
    """One merge 'step' plus its algorithmic byte count and dominant kernel family."""

    name = ""
    family = ""
    config: dict = {}
    bytes_per_step = 0

    def step(self, index: int) -> None:
        raise NotImplementedError


class Int8Stack(Workload):
    family = "rows_stack"

    def __init__(self, layers: int, stochastic: bool) -> None:
        from piper_offload_amd.stack import StackTarget

        self.plan = None  # descriptor table + workspace, built on the first step
        self.stochastic = stochastic
        self.paths, self.targets = [], []
        rank = 16
        for i in range(layers):
            for name, rows, cols in LAYER_SHAPES:
                path = f"model.layers.{i}.{name}.weight"
                w = _int8_weight(path, rows, cols)
                b, a = _factors(path, rows, cols, rank)
                self.paths.append(path)
                self.targets.append(StackTarget(w, b, a, 1.0, 0))
                self.bytes_per_step += _int8_bytes(rows, cols, rank)
        n_el = sum(t.weight.qdata.numel() for t in self.targets)
        self.name = "int8_stack"
        self.config = {
            "workload": f"{layers}-layer 8B-shaped INT8 stack merge ({len(self.targets)} targets: q/o [4096,4096], "
                        "k/v [1024,4096], gate/up [14336,4096], down [4096,14336]); per-row symmetric int8 codes + "
                        "fp32 scales from W~N(0,0.02) (absmax/127); rank-16 bf16 LoRA A~N(0,1/16) B~N(0,0.01), "
                        f"strength 1.0; {'stochastic' if stochastic else 'round-to-nearest'} requant, seed "
                        "derive_seed(param_path, step); one grouped launch per step",
            "targets": len(self.targets), "rank": rank, "elements": n_el,
            "rounding": "stochastic" if stochastic else "nearest",
            "algorithmic_bytes_per_step": self.bytes_per_step,
        }

    def step(self, index: int) -> None:
        from piper_offload_amd import derive_seed

        if self.plan is None:
            from piper_offload_amd.stack import StackPlan

            self.plan = StackPlan(self.targets, "int8")
        self.plan.merge([derive_seed(p, index) for p in self.paths], stochastic=self.stochastic)


class Nvfp4Stack(Workload):
    family = "nvfp4"  # the pruned-amax launches + the quant launch of the two-level merge

    def __init__(self, layers: int, stochastic: bool) -> None:
        from piper_offload_amd.stack import StackTarget

        self.plan = None  # descriptor table + workspace, built on the first step
        self.stochastic = stochastic
        self.paths, self.targets = [], []
        rank = 16
        for i in range(layers):
            for name, rows, cols in LAYER_SHAPES:
                path = f"model.layers.{i}.{name}.weight"
                w = _nvfp4_weight(path, rows, cols)
                b, a = _factors(path, rows, cols, rank)
                self.paths.append(path)
                self.targets.append(StackTarget(w, b, a, 1.0, 0))
                self.bytes_per_step += _nvfp4_bytes(rows, cols, rank)
        self.name = "nvfp4_stack"
        self.config = {
            "workload": f"{layers}-layer 8B-shaped NVFP4 stack merge (two-level: e2m1 codes, e4m3 block-16 scales, "
                        "fp32 per-tensor scale); rank-16 bf16 LoRA, strength 1.0, "
                        f"{'stochastic' if stochastic else 'round-to-nearest'} requant",
            "targets": len(self.targets), "rank": rank,
            "rounding": "stochastic" if stochastic else "nearest",
            "algorithmic_bytes_per_step": self.bytes_per_step,
        }

    def step(self, index: int) -> None:
        from piper_offload_amd import derive_seed

        if self.plan is None:
            from piper_offload_amd.stack import StackPlan

            self.plan = StackPlan(self.targets, "nvfp4")
        self.plan.merge([derive_seed(p, index) for p in self.paths], stochastic=self.stochastic)


class Copy(Workload):
    """Plain device copy (torch elementwise kernel, 1 GiB in + 1 GiB out): the achievable-HBM reference
    and the byte-counter calibration for the rocprofv3 FETCH_SIZE / WRITE_SIZE traffic figures."""

    family = ""

    def __init__(self) -> None:
        import torch

        n = 1 << 28  # int32 elements = 1 GiB
        self.src = torch.arange(n, device="cuda", dtype=torch.int32)
        self.dst = torch.empty_like(self.src)
        self.bytes_per_step = 2 * self.src.numel() * 4
        self.name = "copy"
        self.config = {"workload": "device copy 1 GiB -> 1 GiB (torch.bitwise_not on int32)",
                       "algorithmic_bytes_per_step": self.bytes_per_step}

    def step(self, index: int) -> None:
        import torch

        torch.bitwise_not(self.src, out=self.dst)


class _HostStack:
    """The 8B-shaped INT8 stack with its stored weights in pinned host memory
    (what an offloaded model keeps between reloads) and its factors on the GPU."""

    def __init__(self, layers: int) -> None:
        from piper_offload_amd.reload import HostInt8Target

        self.layers = []
        self.h2d_bytes = 0
        for layer in range(layers):
            targets = []
            for name, rows, cols in LAYER_SHAPES:
                path = f"model.layers.{layer}.{name}.weight"
                w = _int8_weight(path, rows, cols)
                b, a = _factors(path, rows, cols, 16)
                targets.append(HostInt8Target(path, w.qdata.cpu().pin_memory(), w.scale.cpu().pin_memory(), b, a, 1.0))
                self.h2d_bytes += w.qdata.numel() + 4 * w.scale.numel()
                del w
            self.layers.append(targets)


class Reload(Workload):
    """Merge on reload (P/model_offloader.py:245-288): every step reloads all
    layers of the stack from pinned host memory through two device slots and
    merges each layer (one grouped launch) while the next layer is copied."""

    family = "rows_stack"

    def __init__(self, layers: int, stochastic: bool) -> None:
        from piper_offload_amd.reload import ReloadMergePipeline

        host = _HostStack(layers)
        self.pipe = ReloadMergePipeline(host.layers, slots=2, stochastic=stochastic)
        self.n = len(host.layers)
        self.bytes_per_step = host.h2d_bytes
        # the merge kernels' own algorithmic bytes, for the roofline block
        self.kernel_bytes_per_step = layers * sum(_int8_bytes(r, c, 16) for _, r, c in LAYER_SHAPES)
        self.name = "reload"
        self.config = {"workload": f"{layers}-layer 8B-shaped INT8 stack reloaded from pinned host memory and merged "
                                   f"on reload (copy stream + merge stream, 2 device slots, one grouped merge per "
                                   f"layer, {'stochastic' if stochastic else 'round-to-nearest'} requant, seed "
                                   f"derive_seed(param_path, step)); value = host-to-device GB/s of the stored weights",
                       "h2d_bytes_per_step": self.bytes_per_step}

    def step(self, index: int) -> None:
        for layer in range(self.n):
            r = self.pipe.reload(layer, index)
            r.wait()  # the consumer (the current stream) uses the merged layer ...
            self.pipe.release(r)  # ... and hands the slot back


class H2D(Workload):
    """The reload workload's copies alone (same bytes, same two slots, one
    stream, no merge): the host-link baseline the merge hides behind."""

    family = ""

    def __init__(self, layers: int) -> None:
        import torch

        host = _HostStack(layers)
        self.layers = host.layers
        self.slots = [[(torch.empty_like(t.qdata, device="cuda"), torch.empty_like(t.scale, device="cuda"))
                       for t in self.layers[0]] for _ in range(2)]
        self.bytes_per_step = host.h2d_bytes
        self.name = "h2d"
        self.config = {"workload": f"{layers}-layer 8B-shaped INT8 stack copied from pinned host memory (no merge)",
                       "h2d_bytes_per_step": self.bytes_per_step}

    def step(self, index: int) -> None:
        for layer, targets in enumerate(self.layers):
            for (q, s), t in zip(self.slots[layer % 2], targets):
                q.copy_(t.qdata, non_blocking=True)
                s.copy_(t.scale, non_blocking=True)


class Api(Workload):
    """The 8B-shaped INT8 stack merged through the drop-in API, ``merge_lora(model, [(lora, 1.0)])``
    (P/merge.py:54-87): a module whose 224 weights are INT8 tensors on the GPU and a LoRA whose factors
    sit in pinned host memory, so every step resolves the targets, stages each target's factors with
    one host-to-device copy and merges them with one grouped launch."""

    family = "rows_stack"

    def __init__(self, layers: int, stochastic: bool) -> None:
        from torch import nn

        from piper_offload_amd import LoRA

        self.stochastic = stochastic
        self.model = nn.Module()
        sd = {}
        rank = 16
        for i in range(layers):
            for name, rows, cols in LAYER_SHAPES:
                path = f"model.layers.{i}.{name}.weight"
                key = f"layers_{i}_{name.replace('.', '_')}"  # one holder module per weight: parameter '<key>.weight'
                holder = nn.Module()
                holder.weight = nn.Parameter(_int8_weight(path, rows, cols), requires_grad=False)
                self.model.add_module(key, holder)
                b, a = _factors(path, rows, cols, rank)
                sd[f"{key}.lora_A.weight"] = a.cpu()
                sd[f"{key}.lora_B.weight"] = b.cpu()
                self.bytes_per_step += _int8_bytes(rows, cols, rank)
        self.lora = LoRA.from_state_dict(sd)
        self.name = "api"
        self.config = {"workload": f"{layers}-layer 8B-shaped INT8 stack ({7 * layers} targets) merged by "
                                   "merge_lora(model, [(lora, 1.0)]): factors in pinned host memory, staged once per "
                                   "target, one grouped merge launch, "
                                   f"{'stochastic' if stochastic else 'round-to-nearest'} requant",
                       "targets": 7 * layers, "rank": rank, "algorithmic_bytes_per_step": self.bytes_per_step}

    def step(self, index: int) -> None:
        from piper_offload_amd import merge_lora

        merge_lora(self.model, [(self.lora, 1.0)], stochastic_rounding=self.stochastic)


class Routed(Workload):
    """Routed LoRA residual (P/lora.py:801-829) after a gate_proj-shaped Linear: tokens x 4096 -> 14336, rank 16,
    bf16: out = y + ((x A^T) s) B^T, one down-projection and one up-projection launch per step."""

    family = "routed"

    def __init__(self, tokens: int) -> None:
        import torch

        from piper_offload_amd.routed import RoutedFactor

        K, N, rank = 4096, 14336, 16
        self.x = _normal((tokens, K), 1.0, 11)
        self.y = _normal((tokens, N), 0.5, 12)
        self.f = [RoutedFactor(_normal((rank, K), 1.0 / rank, 13), _normal((N, rank), 0.01, 14), 1.0)]
        self.bytes_per_step = 2 * (tokens * K + 2 * tokens * N + rank * (K + N))
        self.name = "routed"
        self.config = {"workload": f"routed LoRA residual, {tokens} tokens x [4096 -> 14336] (gate_proj), rank 16, "
                                   "bf16: reads x, y, A, B once, writes out once",
                       "tokens": tokens, "rank": rank, "algorithmic_bytes_per_step": self.bytes_per_step}
        torch.cuda.synchronize()

    def step(self, index: int) -> None:
        import torch

        from piper_offload_amd.routed import routed_residual

        with torch.no_grad():
            self.out = routed_residual(self.x, self.f, self.y)


class Gguf(Workload):
    """GGUF dequantize (P/gguf_dequant.py:303-331) of one gate_proj-shaped [14336, 4096] tensor to bf16."""

    family = "gguf"

    def __init__(self, type_name: str) -> None:
        import torch

        from piper_offload_amd.gguf_dequant import GGML_QUANT_SIZES

        self.qtype = GGUF_TYPES[type_name]
        rows, cols = 14336, 4096
        raw = _gguf_bytes(self.qtype, rows, cols, 0)
        self.data = torch.from_numpy(raw).to("cuda")
        self.out_bytes = 2 * rows * cols
        self.bytes_per_step = raw.size + self.out_bytes
        self.name = f"gguf_{type_name.lower()}"
        bs, ts = GGML_QUANT_SIZES[self.qtype]
        self.config = {"workload": f"GGUF {type_name} dequantize [{rows},{cols}] -> bf16 ({ts} B per {bs} elements)",
                       "quant_type": type_name, "algorithmic_bytes_per_step": self.bytes_per_step}

    def step(self, index: int) -> None:
        from piper_offload_amd.gguf_dequant import dequantize

        dequantize(self.data, self.qtype)


class Single(Workload):
    """One tensor of configs 2-4 (or NVFP4 / MXFP4 at the gate_proj shape)."""

    def __init__(self, kind: str, stochastic: bool) -> None:
        import torch

        from piper_offload_amd import derive_seed
        from piper_offload_amd import kernels as K

        self.kind, self.stochastic = kind, stochastic
        self.path = "bench.weight"
        if kind == "int8":
            rows, cols, rank, self.strength = 14336, 4096, 32, 0.5
            w = _int8_weight(self.path, rows, cols)
            self.q, self.s = w.qdata, w.scale
            self.family = "rows"
            self.bytes_per_step = _int8_bytes(rows, cols, rank)
        elif kind == "fp8":
            rows, cols, rank, self.strength = 8192, 8192, 64, 1.0
            w = _normal((rows, cols), 0.02, derive_seed(self.path, 0)).float()
            self.s = (w.abs().amax(dim=1, keepdim=True) / 448.0).clamp_min(torch.finfo(torch.float32).eps)
            self.q = (w / self.s).clamp_(-448, 448).to(torch.float8_e4m3fn)
            self.family = "rows"
            self.bytes_per_step = 2 * rows * cols + 8 * rows + 2 * rank * (rows + cols)
        elif kind == "q8_0":
            rows, cols, rank, self.strength = 13824, 5120, 16, 1.0
            self.q = K.requantize_q8_0(_normal((rows, cols), 0.02, derive_seed(self.path, 0)))
            self.family = "q8"
            self.bytes_per_step = 2 * rows * (cols // 32 * 34) + 2 * rank * (rows + cols)
        elif kind == "nvfp4":
            rows, cols, rank, self.strength = 14336, 4096, 16, 1.0
            self.w = _nvfp4_weight(self.path, rows, cols)
            self.family = "nvfp4"
            self.bytes_per_step = _nvfp4_bytes(rows, cols, rank)
        else:  # mxfp4
            rows, cols, rank, self.strength = 14336, 4096, 16, 1.0
            q, s = K.requantize_mx(_normal((rows, cols), 0.02, derive_seed(self.path, 0)), torch.float4_e2m1fn_x2)
            self.q, self.s = q, s
            self.family = "mx"
            self.bytes_per_step = 2 * (rows * cols // 2 + rows * cols // 32) + 2 * rank * (rows + cols)
        self.b, self.a = _factors(self.path, rows, cols, rank)
        self.name = kind
        self.config = {"workload": f"{kind} merge [{rows},{cols}] rank {rank} strength {self.strength}, "
                                   f"{'stochastic' if stochastic else 'round-to-nearest'} requant",
                       "rank": rank, "rounding": "stochastic" if stochastic else "nearest",
                       "algorithmic_bytes_per_step": self.bytes_per_step}

    def step(self, index: int) -> None:
        import torch

        from piper_offload_amd import derive_seed
        from piper_offload_amd import kernels as K

        seed = derive_seed(self.path, index) if self.stochastic else None
        if self.kind == "int8":
            K.merge_int8_lora_into(self.q, self.s, None, (1, self.q.shape[1]), self.b, self.a, self.strength,
                                   asymmetric=False, reduce_range=False, rounding_seed=seed, out_qdata=self.q,
                                   out_scale=self.s, out_zero_point=None)
        elif self.kind == "fp8":
            K.merge_float8_lora_into(self.q, self.s, (1, self.q.shape[1]), self.b, self.a, self.strength,
                                     rounding_seed=seed, out_qdata=self.q, out_scale=self.s)
        elif self.kind == "q8_0":
            K.merge_q8_0_lora(self.q, self.b, self.a, self.strength, rounding_seed=seed, out=self.q)
        elif self.kind == "nvfp4":
            w = self.w
            K.merge_nvfp4_lora_into(w.qdata, w.scale, w.per_tensor_scale, 16, False, self.b, self.a, self.strength,
                                    rounding_seed=seed, out_qdata=w.qdata, out_scale=w.scale,
                                    out_per_tensor_scale=w.per_tensor_scale)
        else:
            K.merge_mx_lora_(self.q, self.s, torch.float4_e2m1fn_x2, 32, torch.bfloat16, self.b, self.a,
                             self.strength, scaling_mode=0, swizzled=False, rounding_seed=seed)


# ---------------------------------------------------------------------------
# CPU baseline: the reference's portable path in torch CPU ops, bounded sample
# ---------------------------------------------------------------------------
def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(kind: str, stochastic: bool, budget_s: float, gguf_type: str = "Q4_K") -> dict | None:
    """Time the CPU path on the host cores, on a bounded sample of the workload.

    Merge workloads run the reference's portable merge of their format
    (dequantize, addmm_, requantize; oracle/portable.py) with torch CPU ops on
    every core of this process's affinity (the reference's own CPU fallback) on
    one tensor of the workload's shape: INT8 (stacks, reload, api), FP8, NVFP4
    (single and stack), MXFP4, Q8_0.  GGUF runs the oracle's dequantize (C,
    OpenMP); routed runs the residual in torch CPU ops; copy and h2d a torch CPU
    copy of the same bytes.  One warm-up, then repeats until the budget is spent
    (at least 3), and the median repeat is reported.
    """
    if budget_s <= 0:
        return None
    import statistics

    import torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    from piper_offload_amd import derive_seed

    path = "model.layers.0.mlp.gate_proj.weight"
    rows, cols = 14336, 4096
    if kind in ("int8_stack", "int8", "api", "reload"):
        from oracle import portable as P

        rank, strength = (32, 0.5) if kind == "int8" else (16, 1.0)
        g = torch.Generator(device="cpu").manual_seed(derive_seed(path, 0) % (1 << 63))
        w = torch.randn((rows, cols), generator=g) * 0.02
        scale = (w.abs().amax(dim=1, keepdim=True) / 127.0).clamp_min(torch.finfo(torch.float32).eps)
        q = torch.round(w / scale).clamp_(-128, 127).to(torch.int8)
        del w
        a = (torch.randn((rank, cols), generator=g) / rank).to(torch.bfloat16)
        b = (torch.randn((rows, rank), generator=g) * 0.01).to(torch.bfloat16)
        seeds = iter(range(1 << 30))

        def run() -> None:
            P.int8_merge(q, scale, b, a, strength,
                         rounding_seed=derive_seed(path, next(seeds)) if stochastic else None)

        nbytes = _int8_bytes(rows, cols, rank)
        what = (f"reference portable path in torch CPU ops (dequantize, addmm_, requantize, "
                f"{'stochastic' if stochastic else 'round-to-nearest'}) of one {rows} x {cols} gate_proj-shaped "
                f"INT8 tensor, rank {rank}")
    elif kind in ("fp8", "nvfp4", "nvfp4_stack", "mxfp4", "q8_0"):
        from oracle import portable as P

        if kind == "fp8":
            rows, cols, rank, strength, label = 8192, 8192, 64, 1.0, "config-3 [8192, 8192] e4m3fn per-row"
        elif kind == "q8_0":
            rows, cols, rank, strength, label = 13824, 5120, 16, 1.0, "config-4 [13824, 5120] GGUF Q8_0"
        else:
            rank, strength = 16, 1.0
            label = f"{rows} x {cols} gate_proj-shaped " + ("MXFP4 (FLOOR scales)" if kind == "mxfp4" else
                                                          "two-level NVFP4")
        g = torch.Generator(device="cpu").manual_seed(derive_seed(path, 0) % (1 << 63))
        w = (torch.randn((rows, cols), generator=g) * 0.02).to(torch.bfloat16)
        a = (torch.randn((rank, cols), generator=g) / rank).to(torch.bfloat16)
        b = (torch.randn((rows, rank), generator=g) * 0.01).to(torch.bfloat16)
        seeds = iter(range(1 << 30))

        def seed() -> int | None:
            return derive_seed(path, next(seeds)) if stochastic else None

        if kind == "fp8":
            q, sc = P.fp8_requant(w)

            def run() -> None:
                P.fp8_merge(q, sc, b, a, strength, rounding_seed=seed())

            nbytes = 2 * rows * cols + 8 * rows + 2 * rank * (rows + cols)
        elif kind == "q8_0":
            pk = P.q8_0_requant(w)

            def run() -> None:
                P.q8_0_merge(pk, cols, b, a, strength, rounding_seed=seed())

            nbytes = 2 * rows * (cols // 32 * 34) + 2 * rank * (rows + cols)
        elif kind == "mxfp4":
            q, sc = P.mxfp4_requant(w)

            def run() -> None:
                P.mxfp4_merge(q, sc, b, a, strength, rounding_seed=seed())

            nbytes = 2 * (rows * cols // 2 + rows * cols // 32) + 2 * rank * (rows + cols)
        else:
            q, sc, gs = P.nvfp4_requant(w)

            def run() -> None:
                P.nvfp4_merge(q, sc, gs, b, a, strength, rounding_seed=seed())

            nbytes = _nvfp4_bytes(rows, cols, rank)
        del w
        what = (f"reference portable path in torch CPU ops (dequantize, addmm_, requantize, "
                f"{'stochastic' if stochastic else 'round-to-nearest'}) of one {label} tensor, rank {rank}")
    elif kind == "routed":
        tokens, K_, N_, rank = 4096, 4096, 14336, 16
        g = torch.Generator(device="cpu").manual_seed(11)
        x = torch.randn((tokens, K_), generator=g).to(torch.bfloat16)
        y = (torch.randn((tokens, N_), generator=g) * 0.5).to(torch.bfloat16)
        a = (torch.randn((rank, K_), generator=g) / rank).to(torch.bfloat16)
        b = (torch.randn((N_, rank), generator=g) * 0.01).to(torch.bfloat16)

        def run() -> None:
            # P/lora.py:801-829: y + strength * ((x A^T) B^T), torch CPU ops
            torch.addmm(y, x @ a.t(), b.t(), alpha=1.0)

        nbytes = 2 * (tokens * K_ + 2 * tokens * N_ + rank * (K_ + N_))
        what = f"routed residual y + (x A^T) B^T in torch CPU ops, {tokens} tokens x [4096 -> 14336], rank 16"
    elif kind in ("copy", "h2d"):
        src = torch.empty(1 << 28, dtype=torch.int32)
        src.fill_(7)
        dst = torch.empty_like(src)

        def run() -> None:
            dst.copy_(src)

        nbytes = 2 * src.numel() * 4
        what = "torch CPU copy 1 GiB -> 1 GiB"
    elif kind == "gguf":
        import oracle as O

        qtype = GGUF_TYPES[gguf_type]
        data = _gguf_bytes(qtype, rows, cols, 1)
        from piper_offload_amd.gguf_dequant import GGML_QUANT_SIZES

        bs, ts = GGML_QUANT_SIZES[qtype]

        def run() -> None:
            O.gguf_dequant(data, qtype, cd=O.DT_BF16)

        nbytes = rows * cols * 2 + rows * cols // bs * ts
        what = f"oracle GGUF dequantize (C, OpenMP) of one {rows} x {cols} {gguf_type} tensor to bf16"
    else:
        return None
    run()  # warm-up: first touch of the buffers and the thread pool
    times: list[float] = []
    t_start = time.perf_counter()
    while len(times) < 3 or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "cpu": _cpu_model(), "ms_per_merge": round(med * 1e3, 1),
            "sample": f"{what}: median of {len(times)} repeats after one warm-up ({sum(times):.1f} s)"}


def _limiter(name: str, stochastic: bool) -> dict | None:
    """What the counters say limits the dominant kernel below its roofline, from the
    committed counter summary of this workload (profiles/<name>_counters.json)."""
    path = os.path.join(ROOT, "profiles", f"{name}_counters.json")
    try:
        with open(path) as f:
            rec = json.load(f)
        if "stochastic" in rec and bool(rec["stochastic"]) != stochastic:
            return None
        return {"limiter": rec["limiter"], "evidence": rec["evidence"], "source": f"profiles/{name}_counters.json"}
    except (OSError, KeyError, ValueError):
        return None


def _traffic(name: str, kbytes: int, stochastic: bool) -> int | None:
    """Measured HBM bytes per launch, only for the configuration they were measured on.

    A record applies when its algorithmic bytes equal this run's (same shapes,
    layers, tokens) and, where it names one, its rounding mode matches.
    """
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
        if int(rec["algorithmic_bytes_per_launch"]) != int(kbytes):
            return None
        if "stochastic" in rec and bool(rec["stochastic"]) != stochastic:
            return None
        return int(rec["hbm_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def main() -> int:
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the merge shards by weight and by row "
              "with no exchange except one scalar max for two-level scales; run it on one GPU per shard",
              file=sys.stderr)
        return 2
    import torch

    from piper_offload_amd import _lib as L

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    L.lib()
    stochastic = args.rounding == "stochastic"
    print(f"[bench] building workload {args.workload} ...", file=sys.stderr, flush=True)
    if args.workload == "int8_stack":
        wl: Workload = Int8Stack(args.layers, stochastic)
    elif args.workload == "copy":
        wl = Copy()
    elif args.workload == "nvfp4_stack":
        wl = Nvfp4Stack(args.layers, stochastic)
    elif args.workload == "gguf":
        wl = Gguf(args.gguf_type)
    elif args.workload == "reload":
        wl = Reload(args.layers, stochastic)
    elif args.workload == "h2d":
        wl = H2D(args.layers)
    elif args.workload == "api":
        wl = Api(args.layers, stochastic)
    elif args.workload == "routed":
        wl = Routed(args.tokens)
    else:
        wl = Single(args.workload, stochastic)
    torch.cuda.synchronize()
    print(f"[bench] warmup {args.warmup} ...", file=sys.stderr, flush=True)
    for i in range(args.warmup):
        wl.step(i)
    torch.cuda.synchronize()
    # Two timed regions of K steps each.  The first gives ms_per_step and
    # `value` with nothing between the launches.  The second brackets every
    # launch of the dominant kernel family with HIP events on its stream for
    # `roofline`: those event records sit between the launches and cost
    # ~20 us per step (measured), a third of a single-tensor merge.
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for i in range(args.steps):
        wl.step(args.warmup + i)
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = start.elapsed_time(stop)
    kern_ms, launches = ev_ms, args.steps
    if wl.family:
        L.timer_enable(True)
        for i in range(args.steps):
            wl.step(args.warmup + args.steps + i)
        torch.cuda.synchronize()
        kern_ms, launches = L.timer_read(wl.family)
        L.timer_enable(False)
    ms_per_step = ev_ms / args.steps
    value = wl.bytes_per_step / (ms_per_step * 1e-3) / 1e9
    print(f"[bench] {args.steps} steps: {ms_per_step:.3f} ms/step (events), wall {wall / args.steps * 1e3:.3f} ms/step, "
          f"{wl.family}: {launches} launches {kern_ms / max(launches, 1):.3f} ms avg", file=sys.stderr, flush=True)
    # the dominant kernel family's time per step (one launch, or the amax +
    # quant launches of a two-level NVFP4 merge) against the step's bytes
    kbytes = getattr(wl, "kernel_bytes_per_step", wl.bytes_per_step)
    achieved = kbytes * args.steps / (kern_ms * 1e-3) / 1e9 if launches else None
    print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
    cpu = cpu_baseline(args.workload, stochastic, args.cpu_seconds, args.gguf_type)
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": wl.config,
        "hbm_peak_fraction": round(value / HBM_PEAK_GBS, 4),
        # bound: the roofline the kernel is measured against (HBM: the merge's
        # arithmetic intensity, 2r flops per 2 bytes, is far below the MFMA
        # ridge of 2.5 PFLOP/s / 8 TB/s); limiter: what the counters say stops
        # it short of that roofline
        "roofline": {
            "bound": "hbm",
            **(_limiter(wl.name, stochastic) or {}),
            "kernel": wl.family,
            "kernel_ms": None if not launches else round(kern_ms / launches, 4),
            "achieved": None if achieved is None else round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": None if achieved is None else round(achieved / HBM_PEAK_GBS, 4),
            "traffic": _traffic(wl.name, kbytes, stochastic),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
