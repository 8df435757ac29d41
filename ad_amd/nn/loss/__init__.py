"""Categorical cross-entropy built from graph primitives
(autodiff/nn/loss/categorical.py:3-25)."""

__all__ = ["categorical_cross_entropy"]


def categorical_cross_entropy(logits, one_hot_labels):
    shifted_logits = logits - logits.max(1).unsqueeze(1)
    exp_vals = shifted_logits.exp()
    softmax_probs = exp_vals / exp_vals.sum(1).unsqueeze(1)
    log_probs = softmax_probs.ln()
    correct_logprobs = -1 * (one_hot_labels * log_probs).sum(1).unsqueeze(1)
    return correct_logprobs.mean(-1)
