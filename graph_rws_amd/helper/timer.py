"""SpMM time list and the per-batch stage timer (helper/timer.py:1-90 of the
reference).

The reference appends the per-call kernel ms that spmm_tc returns.  Here
spmm_tc reports 0.0 unless graph_rws_amd.core.ops.TIMING is set (timing a
call costs a stream synchronisation), so the average stays 0 in the
default, unsynchronised configuration.
"""
from __future__ import annotations

import time

_SPMM_TIMINGS: list = []


def record_spmm_time(t: float) -> None:
    """Called by BCSRSPMMFunction with the ms of one SpMM (timer.py:9-11)."""
    _SPMM_TIMINGS.append(float(t))


def reset_spmm_timings() -> None:
    _SPMM_TIMINGS.clear()


def get_avg_spmm_time() -> float:
    if not _SPMM_TIMINGS:
        return 0.0
    return sum(_SPMM_TIMINGS) / len(_SPMM_TIMINGS)


# earlier names of this module, kept for callers written against them
def get_spmm_time() -> float:
    return sum(_SPMM_TIMINGS)


def reset_spmm_time() -> None:
    reset_spmm_timings()


class EpochTimer:
    """Average wall ms per batch of the stages Data, Sample, Fwd, Bwd, Step
    (timer.py:49-90).  Host clock only: a stage that ends in queued GPU work
    is charged to the stage that next waits for the device."""

    def __init__(self):
        self.keys = ["Data", "Sample", "Fwd", "Bwd", "Step"]
        self.reset()

    def reset(self):
        self.metrics = {k: 0.0 for k in self.keys}
        self.counts = 0
        self.t_mark = 0.0
        reset_spmm_timings()

    def start_batch(self):
        self.t_mark = time.time()

    def record(self, key: str):
        now = time.time()
        self.metrics[key] += now - self.t_mark
        self.t_mark = now

    def end_batch(self):
        self.counts += 1

    def get_epoch_stats(self) -> dict:
        spmm = get_avg_spmm_time()
        if self.counts == 0:
            stats = {k: 0.0 for k in self.metrics}
        else:
            stats = {k: v / self.counts * 1000.0 for k, v in self.metrics.items()}
        stats["SpMM"] = spmm
        return stats
