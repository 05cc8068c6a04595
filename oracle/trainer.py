"""CPU restatement of the trainer's per-batch metrics on the PADDED batch.  TEST INFRASTRUCTURE
ONLY: imported by tests/, never by the product path.

solution/fast_qwen.py:803-871 (packing) and 1551-1565 (batch_metrics) read the per-token stats
through the packing's permutation; this restatement reads them per padded row and position
instead, with plain loops, so that the packing's order, its targets and the metric formulas are
checked against an independent walk of the batch:
    token (b, t), t < len_b, is real; its target is labels[b, t + 1] when t + 1 < T and that label
    is not -100 (ignore index), else it has none
    entropy  = sum over real tokens of their entropy / number of real tokens
    accuracy = sum over tokens with a target of hit / their number (0 without any)
    row_loss = per row, the mean loss over its tokens with a target (0 without any)
"""

import numpy as np


def padded_metrics(stats_of, lens, labels):
    """stats_of(b, t) -> (loss, entropy, hit) of real token (b, t); lens [B]; labels [B, T]."""
    labels = np.asarray(labels)
    B, T = labels.shape
    ent_sum, n_real, hits, n_lab = 0.0, 0, 0.0, 0
    row_loss, row_tokens = [], []
    for b in range(B):
        loss_b, cnt_b = 0.0, 0
        for t in range(int(lens[b])):
            loss, ent, hit = stats_of(b, t)
            ent_sum += float(ent)
            n_real += 1
            if t + 1 < T and labels[b, t + 1] != -100:
                hits += float(hit)
                n_lab += 1
                loss_b += float(loss)
                cnt_b += 1
        row_loss.append(loss_b / cnt_b if cnt_b else 0.0)
        row_tokens.append(cnt_b)
    return {"entropy": ent_sum / n_real, "accuracy": hits / n_lab if n_lab else 0.0,
            "n_lab": n_lab, "row_loss": row_loss, "row_tokens": row_tokens}
