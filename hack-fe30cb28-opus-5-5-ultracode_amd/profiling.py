"""Per-launch timing of one C-ABI entry point with HIP events, and its algorithmic work.

`LaunchTimer(entry)` times each launch of `entry` while active with a pair of HIP events on
torch's current stream (the stream every entry point is launched on): recorded by the kernel
dispatch itself at the kernel's start and end where the entry has a timed form (the dequant, the
package GEMM), else around the call, behind a short spin kernel that keeps the GPU busy while
the host enqueues the events and the launch (so the events bracket the launch's own GPU time,
not the host's Python and ctypes overhead; the dispatch gap between the kernels of a multi-kernel
entry stays in). It reports the average launch duration and the achieved bandwidth or FLOP rate
against the MI355X peak (HBM 8 TB/s, dense fp16 MFMA 2.5 PFLOP/s).
"""

import torch

from . import _lib

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
# GPU clock cycles of the spin kernel ahead of an event-bracketed launch (about 100 us, well
# above the host's time to record an event and enqueue one entry point's kernels)
COVER_CYCLES = 200_000

# the entry point of the step's largest hand-written kernel by time, the package's MFMA GEMM
# (every projection and lm_head product; the roofline entry is its gate|up forward with the
# SwiGLU epilogue); the dequant, the north star's "NF4 dequant HBM GB/s", is reported beside it
DOMINANT = "qlora_gemm16"
DEQUANT = "qlora_nf4_dequant_many"

# Measured HBM bytes per launch over algorithmic bytes per launch: rocprofv3 FETCH_SIZE and
# WRITE_SIZE of the layer-wide dequant launch (the same kernel and byte count as each of the
# step's launches), each divided by what the counter reads for a plain device copy of 1 GiB
# (512 MiB each way; FETCH 0.50004, WRITE 1.000 of the bytes moved):
# (11,892.4 / 0.50004 + 91,392) KiB per launch = 1.0018 x the algorithmic 117,728,444 B.
# The package GEMM's SwiGLU products that keep [g | u] (hgemm_kernel<NT, epilogue 5> with the
# automatic plan: one launch, or whole 256 x 256 rounds and the remaining columns on 128 x 128
# tiles) over the step's products of the bench's four measuring batches: 2.030 x the
# algorithmic bytes (x, the [gate; up] weight, m and [g | u] once each), weighted by product;
# 1.85-2.34 per token count. WRITE equals the outputs; the excess is in FETCH, the A rows and
# B tiles fetched by each XCD that uses them (FETCH_SIZE counts what leaves the 4 MB L2,
# Infinity Cache hits included).
TRAFFIC_RATIO = {"qlora_nf4_dequant_many": 1.0018, "qlora_gemm16": 2.030}


def _dequant_bytes(args):
    """Algorithmic HBM bytes of one qlora_nf4_dequant launch: packed nibbles, absmax, the
    double-quantisation tables, and the fp16 output."""
    n_blocks, nested, bs1, bs2, seg1, seg2 = args[7], args[8], args[10], args[11], args[12], \
        args[13]
    numel = n_blocks * bs1
    b = numel // 2 + 2 * numel
    if nested:
        segs = 1 + (seg1 < n_blocks) + (seg2 < n_blocks)
        b += n_blocks + 4 * ((n_blocks + bs2 - 1) // bs2) + 4 * 256 + 4 * segs
    else:
        b += 4 * n_blocks
    return b


def _dequant_many_bytes(args):
    """The same, summed over the weights of one qlora_nf4_dequant_many launch."""
    k = args[0]
    total = 0
    for i in range(k):
        n_blocks, nested, bs1, bs2 = args[8][i], args[9][i], args[11][i], args[12][i]
        seg1, seg2 = args[13][i], args[14][i]
        total += _dequant_bytes([None] * 7 + [n_blocks, nested, None, bs1, bs2, seg1, seg2])
    return total


# entries with a form that records the events from the kernel dispatch itself
TIMED = {"qlora_nf4_dequant_many": "qlora_nf4_dequant_many_timed",
         "qlora_gemm16": "qlora_gemm16_timed"}


SWIGLU_EPIS = (3, 5)  # the SwiGLU epilogues (5: the product [g | u] written beside it)


def hgemm_flops(args):
    """2 M N K of one qlora_gemm16 launch (a, lda, b, ldb, M, N, K, mode, ..., epi
    at 13): N is the output's columns, I with a SwiGLU epilogue, whose product is [M, 2 I]."""
    return 2.0 * args[4] * args[5] * args[6] * (2 if args[13] in SWIGLU_EPIS else 1)


def hgemm_bytes(args):
    """Algorithmic HBM bytes of one qlora_gemm16 launch: A [M, K], the weight
    ([N, K], [2 I, K] with a SwiGLU epilogue, [K, N] in NN) and the fp16 output [M, N] once
    each, and with epilogue 5 the product [g | u] [M, 2 I] written beside it."""
    M, N, K, epi = args[4], args[5], args[6], args[13]
    b = 2.0 * (M * K + (2 * N if epi in SWIGLU_EPIS else N) * K + M * N)
    return b + (2.0 * M * 2 * N if epi == 5 else 0.0)

WORK = {
    "qlora_nf4_dequant": ("hbm", _dequant_bytes),
    "qlora_nf4_dequant_many": ("hbm", _dequant_many_bytes),
}


class LaunchTimer:
    """Times every launch of `entry` while active. The work of a launch comes from WORK, or
    from `work` (a function of the call's arguments) with its `bound` ("hbm": bytes, "mfma":
    flops), or is given afterwards per launch to summary() (`work_total`). `nbytes`: the
    algorithmic HBM bytes of a launch of an MFMA-bound entry (the base of its measured traffic)."""

    def __init__(self, entry, work=None, bound=None, nbytes=None):
        if work is None and bound is None and entry not in WORK:
            raise ValueError(f"no work model for {entry}")
        self.entry = entry
        self.bound, self.work = WORK.get(entry, (bound, work))
        if work is not None:
            self.bound, self.work = bound, work
        if self.work is None:
            self.work = lambda args: 0.0
        self.nbytes = nbytes
        self.records = []

    def __enter__(self):
        _lib.HOOKS[self.entry] = self
        return self

    def __exit__(self, *exc):
        _lib.HOOKS.pop(self.entry, None)
        return False

    def call(self, fn, args):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        timed = TIMED.get(self.entry)
        if timed is not None:
            # the dispatch records both events at the kernel's own start and end (the records
            # here only create the events)
            start.record()
            end.record()
            rc = getattr(_lib.load(), timed)(*args, start.cuda_event, end.cuda_event)
        else:
            # the GPU spins while the host records the start event and enqueues the launch, so
            # the launch follows the start event at once
            torch.cuda._sleep(COVER_CYCLES)
            start.record()
            rc = fn(*args)
            end.record()
        self.records.append((start, end, self.work(args), args))
        return rc

    def summary(self, work_total=None, select=None, also=()):
        """Average duration and achieved rate over the launches (`select`: a predicate on a
        launch's arguments; `also`: more timers of the same bound whose launches count too)."""
        torch.cuda.synchronize()
        recs = [r for t in (self, *also) for r in t.records if select is None or select(r[3])]
        if not recs:
            return None
        ms = [s.elapsed_time(e) for s, e, _, _ in recs]
        work = sum(w for _, _, w, _ in recs) if work_total is None else work_total
        total_s = sum(ms) * 1e-3
        avg_us = 1e3 * sum(ms) / len(ms)
        if self.bound == "hbm":
            achieved = work / total_s / 1e9
            peak, unit = HBM_PEAK_GBS, "GB/s"
        else:
            achieved = work / total_s / 1e12
            peak, unit = FP16_PEAK_TFLOPS, "TFLOP/s"
        ratio = TRAFFIC_RATIO.get(self.entry)
        traffic = None
        if ratio is not None and self.bound == "hbm":
            traffic = work / len(ms) * ratio
        elif ratio is not None and self.nbytes is not None:
            traffic = sum(self.nbytes(r[3]) for r in recs) / len(recs) * ratio
        return {"bound": self.bound, "achieved": achieved, "peak": peak, "unit": unit,
                "frac": achieved / peak, "traffic": traffic, "kernel": self.entry,
                "launches": len(ms), "avg_us": avg_us,
                "work_per_launch": work / len(ms)}
