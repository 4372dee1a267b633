"""SpMM time accumulator (helper/timer.py:7-19 of the reference).

The reference adds the per-call kernel ms that spmm_tc returns to a global
total.  Here spmm_tc reports 0.0 unless graph_rws_amd.core.ops.TIMING is
set (timing a call costs a stream synchronisation), so the total stays 0
in the default, unsynchronised configuration.
"""
from __future__ import annotations

_total_ms = 0.0


def record_spmm_time(ms: float) -> None:
    global _total_ms
    _total_ms += float(ms)


def get_spmm_time() -> float:
    return _total_ms


def reset_spmm_time() -> None:
    global _total_ms
    _total_ms = 0.0
