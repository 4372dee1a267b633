"""Full-graph training epoch and evaluation (helper/engine.py:22-83, 646-667).

Same steps as the reference: forward over the whole graph, cross-entropy (or
BCE for multi-label) on the training rows, backward, clip_grad_norm_(1.0),
optimizer step, loss.item().  The SpMMs inside run on the gfx950 kernels.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def compute_loss_and_metrics(logits, labels):
    """(loss, correct_count tensor, num_samples) (engine.py:22-41)."""
    if labels.dim() > 1:
        loss = F.binary_cross_entropy_with_logits(logits, labels)
        correct = ((logits > 0).float() == labels).sum()
        return loss, correct, labels.numel()
    loss = F.cross_entropy(logits, labels)
    correct = (logits.argmax(dim=1) == labels).sum()
    return loss, correct, labels.size(0)


def train_epoch_full(model, graphs_for_model, features: torch.Tensor, labels: torch.Tensor,
                     train_idx: torch.Tensor, optimizer: torch.optim.Optimizer, device,
                     timer=None, sync: bool = True):
    """One full-graph training step (engine.py:44-83).  Returns (loss, acc);
    with sync=False the loss and accuracy stay on the device (no host sync)."""
    model.train()
    if timer is not None:
        timer.reset()
    if features.device != device:
        features = features.to(device)
    optimizer.zero_grad()
    logits = model(graphs_for_model, features)
    loss, correct, n = compute_loss_and_metrics(logits[train_idx].float(), labels[train_idx])
    acc = correct / n if n > 0 else 0.0
    loss.backward()
    torch.nn.utils.clip_grad_norm_(model.parameters(), max_norm=1.0)
    optimizer.step()
    if not sync:
        return loss.detach(), acc
    return loss.item(), acc


@torch.no_grad()
def evaluate(model, bcsr_full, features: torch.Tensor, labels: torch.Tensor,
             eval_idx: torch.Tensor, device):
    """Accuracy of a full-graph inference on eval_idx (engine.py:646-667)."""
    model.eval()
    logits = model.inference(bcsr_full, features)
    _, correct, n = compute_loss_and_metrics(logits[eval_idx].float(), labels[eval_idx])
    return (correct / n).item() if n > 0 else 0.0
