"""The five measured workloads (C1-C5) of this backend and their byte models.

Inputs are generated on the CPU with ``torch.Generator().manual_seed(1000 + i)``
(i = config index) and then moved to the GPU, so the GPU kernels, the CPU
checker and the CPU baseline all see bit-identical values.

Algorithmic bytes per launch = bytes every correct implementation must move
from and to HBM: each input read once, each output written once (the
weight/bias vectors and labels included).  For the norm/softmax family this
extends experiments/exp_cliff_roofline.py:229-234 (2 * numel * elt), and adds
the logsumexp and cross-entropy models the reference lacks (:263 "unknown").
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable

import torch

KERNELS = ("layer_norm", "rms_norm", "softmax", "log_softmax", "logsumexp", "cross_entropy")


@dataclass
class Workload:
    key: str                 # e.g. "C2_rms_norm"
    kernel: str              # ViperBench kernel directory
    fn: str                  # unified-API function name
    desc: str
    make: Callable[[], tuple]  # CPU args (positional) for the unified API
    bytes_per_launch: int
    dtype: str
    extra: dict = field(default_factory=dict)


def _gen(index: int) -> torch.Generator:
    return torch.Generator().manual_seed(1000 + index)


def make_c1():
    g = _gen(0)
    x = torch.randn(4096, 1024, generator=g)
    w = 1.0 + 0.1 * torch.randn(1024, generator=g)
    b = 0.1 * torch.randn(1024, generator=g)
    return (x, w, b, 1e-5)


def make_c2():
    g = _gen(1)
    x = torch.randn(8192, 4096, generator=g).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn(4096, generator=g)).to(torch.bfloat16)
    return (x, (4096,), w, 1e-6)


def make_c3():
    g = _gen(2)
    x = 3.0 * torch.randn(16384, 4096, generator=g)
    spikes = torch.rand(16384, 4096, generator=g) < 0.01
    x[spikes] = 20.0
    return (x,)


def make_c4():
    g = _gen(3)
    logits = 2.0 * torch.randn(8192, 32000, generator=g)
    labels = torch.randint(0, 32000, (8192,), generator=g, dtype=torch.int64)
    return (logits, labels, 0.0, 1.0, 0.0, -100, 32000, 0, 32768, False, False)


def make_c5():
    g = _gen(4)
    x = torch.randn(2048, 20480, generator=g).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn(20480, generator=g)).to(torch.bfloat16)
    b = (0.1 * torch.randn(20480, generator=g)).to(torch.bfloat16)
    return (x, w, b, 1e-5)


def _rw(rows, cols, elt, vec_bytes=0):
    return 2 * rows * cols * elt + vec_bytes


WORKLOADS = {
    w.key: w
    for w in [
        Workload("C1_layer_norm", "layer_norm", "layer_norm",
                 "LayerNorm fwd fp32 x[4096,1024], w~N(1,0.1), b~N(0,0.1), eps=1e-5",
                 make_c1, _rw(4096, 1024, 4, 2 * 1024 * 4), "f32"),
        Workload("C2_rms_norm", "rms_norm", "rms_norm",
                 "RMSNorm fwd bf16 x[8192,4096], w~N(1,0.1) [4096] bf16, eps=1e-6",
                 make_c2, _rw(8192, 4096, 2, 4096 * 2), "bf16"),
        Workload("C3_softmax", "softmax", "softmax",
                 "softmax fp32 x[16384,4096]~N(0,3), 1% entries = +20",
                 make_c3, _rw(16384, 4096, 4), "f32"),
        Workload("C3_log_softmax", "log_softmax", "log_softmax",
                 "log_softmax fp32 x[16384,4096]~N(0,3), 1% entries = +20",
                 make_c3, _rw(16384, 4096, 4), "f32"),
        Workload("C3_logsumexp", "logsumexp", "logsumexp",
                 "logsumexp fp32 x[16384,4096]~N(0,3), 1% entries = +20",
                 make_c3, 16384 * 4096 * 4 + 16384 * 4, "f32"),
        Workload("C4_cross_entropy", "cross_entropy", "cross_entropy_fwd",
                 "cross_entropy fwd fp32 logits[8192,32000]~N(0,2), int64 targets, "
                 "BLOCK_SIZE=32768 (one block per row), mean of the 8192 row losses",
                 make_c4, 8192 * 32000 * 4 + 8192 * 8 + 3 * 8192 * 4, "f32"),
        Workload("C5_layer_norm", "layer_norm", "layer_norm",
                 "LayerNorm fwd bf16 x[2048,20480], w~N(1,0.1), b~N(0,0.1), eps=1e-5",
                 make_c5, _rw(2048, 20480, 2, 2 * 20480 * 2), "bf16"),
    ]
}

# the workload BASELINE.json's headline metric is quoted on
HEADLINE = "C2_rms_norm"


def to_device(args: tuple, device) -> tuple:
    return tuple(a.to(device) if isinstance(a, torch.Tensor) else a for a in args)
