from .timer import (  # noqa: F401
    EpochTimer,
    get_avg_spmm_time,
    get_spmm_time,
    record_spmm_time,
    reset_spmm_time,
    reset_spmm_timings,
)
from .engine import (  # noqa: F401
    compute_loss_and_metrics,
    evaluate,
    train_epoch_full,
    train_epoch_node_sampling,
)
from .graphed import GraphedBlockStep, GraphedFullStep, bucket_rows  # noqa: F401
