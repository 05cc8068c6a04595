"""The tensor part of the reference's trainer integration (solution/integration.py:574-677,
solution/fast_qwen.py:803-871, 1551-1565): packing a right-padded Hugging Face batch into the
token stream the QLoRA step runs on, the per-batch metrics from the LM head's per-token
statistics, and the loss normalisation of the trainer's ``compute_loss``.

The surrounding machinery (the Soup/TRL trainer patching, peft, the rewind recorder, deferred
metric threads) is not part of this build: peft, trl and the Soup CLI are not available here, and
none of it is on the NF4 linear path.

    batch = pack(input_ids, attention_mask, labels, vocab)      # or None: not packable
    step = model.QwenQLoRAStep.for_batch(batch, ...)            # the whole step on these tokens
    loss_sum, stats, dy = step.forward()
    loss = compute_loss(loss_sum, batch, num_items_in_batch)
    metrics = batch_metrics(batch, stats.cpu())
"""

from dataclasses import dataclass

import torch


@dataclass
class PackedBatch:
    """A packed batch in the order the step consumes it.

    lens       tokens of each batch row (rows of length 0 are not packable)
    ids        [n] int64 token ids, row after row
    tgt        [n] int64 next-token targets in token order, -1 where there is none
    perm       [n] int64 token order -> sorted order: tokens with a target first
    tgt_sorted [n] tgt[perm]
    row_sorted [n] batch row of each token, sorted order
    valid_sorted [n] bool, token has a target, sorted order
    n_real     n, the number of real (unpadded) tokens
    n_lab      tokens with a target
    B, T       batch rows and padded length
    """
    lens: list
    ids: torch.Tensor
    tgt: torch.Tensor
    perm: torch.Tensor
    tgt_sorted: torch.Tensor
    row_sorted: torch.Tensor
    valid_sorted: torch.Tensor
    n_real: int
    n_lab: int
    B: int
    T: int


def _row_length(mask_row):
    """Real tokens of one right-padded row: n when the row's mask is n ones followed by zeros
    (values other than 0 and 1 do not qualify), else None."""
    n = int(mask_row.count_nonzero())
    if bool((mask_row[:n] == 1).all()) and bool((mask_row[n:] == 0).all()):
        return n
    return None


def pack(input_ids, attention_mask, labels, vocab):
    """Host-side packing of a right-padded batch (the contract of the reference's
    FastQwen2.pack, solution/fast_qwen.py:803-871): the real tokens of each row concatenated; the
    target of a row's token t is the row's label at t + 1 (-1 past the padded length, and every
    negative label, -100 included, means none); tokens with a target first in the sorted order,
    each group in token order.  Returns None when the batch is not exactly packable (the caller
    then uses the stock path): a row whose mask is not a run of ones from its start, an empty row,
    or an id or target outside the vocabulary.

    Rows are walked one at a time (a batch has a handful): each row's run length is validated,
    its ids and targets are sliced out, and the sorted order is a stable sort on "has no
    target"."""
    if input_ids.dim() != 2 or attention_mask.shape != input_ids.shape or labels.shape != input_ids.shape:
        return None
    B, T = input_ids.shape
    ids_rows = input_ids.to("cpu", torch.int64)
    lab_rows = labels.to("cpu", torch.int64)
    mask_rows = attention_mask.to("cpu", torch.int64)
    lens, ids, tgt = [], [], []
    for b in range(B):
        n = _row_length(mask_rows[b])
        if not n:
            return None
        lens.append(n)
        ids.append(ids_rows[b, :n])
        t = torch.full((n,), -1, dtype=torch.int64)
        shifted = lab_rows[b, 1:n + 1]          # T - 1 labels at most: the last token may get none
        t[:shifted.numel()] = shifted
        tgt.append(t.clamp_(min=-1))
    ids, tgt = torch.cat(ids), torch.cat(tgt)
    if int(ids.min()) < 0 or int(ids.max()) >= vocab or int(tgt.max()) >= vocab:
        return None
    rows = torch.repeat_interleave(torch.arange(B, dtype=torch.int64), torch.tensor(lens))
    has = tgt >= 0
    perm = torch.sort((~has).to(torch.int8), stable=True).indices
    return PackedBatch(lens=lens, ids=ids, tgt=tgt, perm=perm, tgt_sorted=tgt[perm],
                       row_sorted=rows[perm], valid_sorted=has[perm], n_real=int(ids.numel()),
                       n_lab=int(has.sum()), B=B, T=T)


def batch_metrics(batch, stats):
    """The trainer's metrics of one packed batch from the head's per-token stats [n, 4] = (loss,
    entropy, hit, lse) in sorted order, on the host (solution/fast_qwen.py:1551-1565):
    entropy = mean over all real tokens, accuracy = hits over tokens with a target, and per batch
    row the mean loss over its tokens with a target and their count.  Sums in float64."""
    st = torch.as_tensor(stats).to("cpu", torch.float64)
    if st.dim() != 2 or st.shape[0] != batch.n_real or st.shape[1] < 3:
        raise ValueError(f"stats must be [{batch.n_real}, 4] in the batch's sorted order")
    valid = torch.as_tensor(batch.valid_sorted, dtype=torch.bool)
    rows = torch.as_tensor(batch.row_sorted, dtype=torch.int64)
    loss_sum = torch.zeros(batch.B, dtype=torch.float64).index_add_(0, rows[valid], st[valid, 0])
    count = torch.bincount(rows[valid], minlength=batch.B)
    return {"entropy": float(st[:, 1].sum()) / batch.n_real,
            "accuracy": float(st[valid, 2].sum()) / batch.n_lab if batch.n_lab else 0.0,
            "n_lab": batch.n_lab,
            "row_loss": [float(s) / max(int(c), 1) for s, c in zip(loss_sum, count)],
            "row_tokens": [int(c) for c in count]}


def compute_loss(loss_sum, batch, num_items_in_batch=None, model_accepts_loss_kwargs=False):
    """The scalar the trainer backpropagates (solution/integration.py:657-664, the Hugging Face
    Trainer's rule): loss_sum / num_items_in_batch when the model takes loss kwargs and the trainer
    passes the item count, else loss_sum over the batch's supervised tokens (at least 1)."""
    if model_accepts_loss_kwargs and num_items_in_batch is not None:
        denom = num_items_in_batch
        if torch.is_tensor(denom):
            denom = denom.to(loss_sum.device)
        return loss_sum / denom
    return loss_sum / max(batch.n_lab, 1)
