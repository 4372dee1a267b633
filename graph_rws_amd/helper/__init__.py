from .timer import record_spmm_time, get_spmm_time, reset_spmm_time  # noqa: F401
from .engine import train_epoch_full, evaluate, compute_loss_and_metrics  # noqa: F401
