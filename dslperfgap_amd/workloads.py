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

KERNELS = ("layer_norm", "rms_norm", "softmax", "log_softmax", "logsumexp", "cross_entropy",
           "argmax", "max_reduction", "mean_reduction")


@dataclass
class Workload:
    key: str                 # e.g. "C2_rms_norm"
    kernel: str              # ViperBench kernel directory
    fn: str                  # unified-API function name
    desc: str
    make: Callable[[], tuple]  # CPU args (positional) for the unified API
    bytes_per_launch: int
    dtype: str
    # measured yardstick: "copy" (reads and writes about as much) or "read"
    # (writes almost nothing)
    peak_kind: str = "copy"
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


def make_c4_bwd():
    """cross_entropy_bwd at C4's shape: the forward's logits and labels, the
    per-row lse of its single column block, and dloss = 1 / n_rows (the
    gradient of the mean of the row losses)."""
    logits, labels = make_c4()[:2]
    lse = torch.logsumexp(logits, dim=1)
    dloss = torch.full((logits.shape[0],), 1.0 / logits.shape[0])
    return (dloss, logits, lse, labels, 0.0, 1.0, 0.0, -100, 32000, 0, 32768, False)


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
                 make_c3, 16384 * 4096 * 4 + 16384 * 4, "f32", "read"),
        Workload("C4_cross_entropy", "cross_entropy", "cross_entropy_fwd",
                 "cross_entropy fwd fp32 logits[8192,32000]~N(0,2), int64 targets, "
                 "BLOCK_SIZE=32768 (one block per row): the row pass (per-row loss, lse, "
                 "z_loss); the scalar mean of the 8192 losses is timed as full_step",
                 make_c4, 8192 * 32000 * 4 + 8192 * 8 + 3 * 8192 * 4, "f32", "read"),
        Workload("C4_cross_entropy_bwd", "cross_entropy", "cross_entropy_bwd",
                 "cross_entropy bwd fp32 logits[8192,32000] (C4's inputs), lse of the forward, "
                 "dloss = 1/8192 per row (gradient of the mean), dlogits fp32",
                 make_c4_bwd, 2 * 8192 * 32000 * 4 + 8192 * 8 + 8192 * 4 + 8192 * 4, "f32"),
        Workload("C5_layer_norm", "layer_norm", "layer_norm",
                 "LayerNorm fwd bf16 x[2048,20480], w~N(1,0.1), b~N(0,0.1), eps=1e-5",
                 make_c5, _rw(2048, 20480, 2, 2 * 20480 * 2), "bf16"),
    ]
}

# BASELINE.json's metric is quoted per kernel, on no single config, so the
# headline (bench.py's default) is the largest config that fits one GPU: C4,
# the cross-entropy forward over 1.05 GB of fp32 logits
HEADLINE = "C4_cross_entropy"


def to_device(args: tuple, device) -> tuple:
    return tuple(a.to(device) if isinstance(a, torch.Tensor) else a for a in args)


# ---------------------------------------------------------------------------
# The reference benchmark's own cases for this family ("small" and "large" per
# kernel, ViperBench/benchmark.py:143-154, 187-198, 232-249, 314-335), with
# the same shapes, dtypes and arguments.  The reference draws them with
# unseeded torch.randn on the GPU; here they come from a seeded CPU generator.
# ---------------------------------------------------------------------------
@dataclass
class RefCase:
    kernel: str
    size: str                 # "small" / "large"
    fn: str
    desc: str                 # the reference's input_desc column
    make: Callable[[], tuple]
    is_slow: bool             # the reference's MEASURE_ITERS_SLOW flag

    @property
    def key(self) -> str:
        return f"{self.kernel}/{self.size}"


def _ref_gen(kernel: str, size: str) -> torch.Generator:
    return torch.Generator().manual_seed(2000 + 2 * KERNELS.index(kernel) + (size == "large"))


def _ce_case(rows, cols, bs, size):
    def make():
        g = _ref_gen("cross_entropy", size)
        logits = torch.randn(rows, cols, generator=g)
        labels = torch.randint(0, cols, (rows,), generator=g, dtype=torch.int64)
        return (logits, labels, 0.0, 1.0, 0.0, -100, cols, 0, bs, False, False)
    return make


def _ln_case(rows, cols, size):
    def make():
        g = _ref_gen("layer_norm", size)
        x = torch.randn(rows, cols, generator=g).to(torch.bfloat16)
        w = torch.randn(cols, generator=g).to(torch.bfloat16)
        b = torch.randn(cols, generator=g).to(torch.bfloat16)
        return (x, w, b)
    return make


def _rms_case(rows, cols, size):
    def make():
        g = _ref_gen("rms_norm", size)
        x = torch.randn(rows, cols, generator=g).to(torch.float16)
        w = torch.randn(cols, generator=g).to(torch.float16)
        return (x, (cols,), w)
    return make


def _x_case(kernel, rows, cols, dtype, size):
    def make():
        g = _ref_gen(kernel, size)
        return (torch.randn(rows, cols, generator=g).to(dtype),)
    return make


def _red_case(kernel, rows, cols, dtype, size):
    def make():
        g = _ref_gen(kernel, size)
        return (torch.randn(rows, cols, generator=g).to(dtype), 1)
    return make


REFERENCE_CASES = [
    RefCase("cross_entropy", "small", "cross_entropy_fwd", "logits:(256,1024) fp32",
            _ce_case(256, 1024, 256, "small"), True),
    RefCase("cross_entropy", "large", "cross_entropy_fwd", "logits:(4096,32768) fp32",
            _ce_case(4096, 32768, 1024, "large"), True),
    RefCase("layer_norm", "small", "layer_norm", "x:(512,1024) bf16", _ln_case(512, 1024, "small"),
            False),
    RefCase("layer_norm", "large", "layer_norm", "x:(8192,8192) bf16",
            _ln_case(8192, 8192, "large"), False),
    RefCase("log_softmax", "small", "log_softmax", "x:(512,1024) fp16",
            _x_case("log_softmax", 512, 1024, torch.float16, "small"), False),
    RefCase("log_softmax", "large", "log_softmax", "x:(4096,32768) fp16",
            _x_case("log_softmax", 4096, 32768, torch.float16, "large"), False),
    RefCase("logsumexp", "small", "logsumexp", "x:(512,1024) fp32",
            _x_case("logsumexp", 512, 1024, torch.float32, "small"), False),
    RefCase("logsumexp", "large", "logsumexp", "x:(8192,16384) fp32",
            _x_case("logsumexp", 8192, 16384, torch.float32, "large"), False),
    RefCase("rms_norm", "small", "rms_norm", "x:(512,1024) w:(1024,) fp16",
            _rms_case(512, 1024, "small"), False),
    RefCase("rms_norm", "large", "rms_norm", "x:(8192,8192) w:(8192,) fp16",
            _rms_case(8192, 8192, "large"), False),
    RefCase("softmax", "small", "softmax", "x:(512,1024) fp16",
            _x_case("softmax", 512, 1024, torch.float16, "small"), False),
    RefCase("softmax", "large", "softmax", "x:(4096,32768) fp16",
            _x_case("softmax", 4096, 32768, torch.float16, "large"), False),
    # sibling row reductions (benchmark.py:89-97, 274-291)
    RefCase("argmax", "small", "argmax", "x:(1024,1024) dim=1 fp16",
            _red_case("argmax", 1024, 1024, torch.float16, "small"), False),
    RefCase("argmax", "large", "argmax", "x:(8192,32768) dim=1 fp16",
            _red_case("argmax", 8192, 32768, torch.float16, "large"), False),
    RefCase("max_reduction", "small", "max_reduction", "x:(1024,1024) dim=1 fp16",
            _red_case("max_reduction", 1024, 1024, torch.float16, "small"), False),
    RefCase("max_reduction", "large", "max_reduction", "x:(8192,32768) dim=1 fp16",
            _red_case("max_reduction", 8192, 32768, torch.float16, "large"), False),
    RefCase("mean_reduction", "small", "mean_reduction", "x:(1024,1024) dim=1 fp32",
            _red_case("mean_reduction", 1024, 1024, torch.float32, "small"), False),
    RefCase("mean_reduction", "large", "mean_reduction", "x:(8192,32768) dim=1 fp32",
            _red_case("mean_reduction", 8192, 32768, torch.float32, "large"), False),
]
