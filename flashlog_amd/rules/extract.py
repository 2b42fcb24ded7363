"""Post-processing of extracted rule candidates (rules/extract.py:37-201,
216-299): attention rank weights, selection, ordering and the rule TSV
lines.

Candidates are int64 rows [length, op_1 .. op_T, walk_hits, source_hits,
positive_walk_hits, positive_source_hits, and the four per-fold minimums]
(the grounding's output, columns -8 .. -1).  The rank weight of a
candidate in channel c is the attention-weighted count of the ways its body
fits into the T steps with the identity elsewhere; the reference's two
evaluations (the 3-step closed form, the dynamic program with sums or
maxima) run in the HIP kernel fl_rule_rank_weights in double precision, op
for op, so the weights are bit-identical to numpy's.  Selection and order
(positive walk hits >= the minimum, else the single best fallback
candidate; then positive source hits descending, weight sum descending,
body ascending, input order) are computed on the GPU by stable sorts.
select_and_annotate_batch does all heads of an attention batch in one
kernel launch.  Inputs and outputs are numpy arrays, as the reference's.
"""
import numpy as np
import torch

from .. import _lib
from .._lib import check, ptr
from ..flashlog_kernel import flashlog_kernel as fk

FIELDS = ("head_id", "body_ids", "length", "weight", "walk_hits", "source_hits", "positive_walk_hits",
          "positive_source_hits", "minimum_fold_walk_hits", "minimum_fold_source_hits",
          "minimum_fold_positive_walk_hits", "minimum_fold_positive_source_hits", "origin", "rank_weights",
          "sampled_train_precision")
SCALAR_FIELDS = ("head_id", "body_ids", "length", "weight", "group_id", "origin")

FALLBACK_CHANNEL_AGGREGATION = "sum"

_CLOSED_FORM, _DP_SUM, _DP_MAX = 0, 1, 2


def _device():
    if not torch.cuda.is_available():
        raise RuntimeError("flashlog_amd rule extraction needs a ROCm GPU")
    return torch.device("cuda", torch.cuda.current_device())


def _attention_tensor(attention, dev, heads_axis):
    """Attention on the GPU as float32 (kept) or float64 (every other float
    type converts exactly), with a leading heads axis."""
    a = torch.as_tensor(np.asarray(attention) if not torch.is_tensor(attention) else attention)
    if a.dtype != torch.float32:
        a = a.to(torch.float64)
    a = a.to(dev).contiguous()
    if not heads_axis:
        a = a.unsqueeze(0)
    if a.dim() != 4:
        raise ValueError("attention must be [steps, channels, operators] (or [heads, ...])")
    return a


def _rows_tensor(rows, dev):
    r = torch.as_tensor(np.asarray(rows) if not torch.is_tensor(rows) else rows).to(device=dev, dtype=torch.int64)
    if r.dim() != 2:
        raise ValueError("candidate rows must be two-dimensional")
    return r.contiguous()


def _annotate(att, rows, row_head, identity, mode, stats=True):
    """(rank weights [N, L], weight sums [N], precision [N]) on the GPU."""
    H, T, L, n = att.shape
    N, W = rows.shape
    dev = rows.device
    rw = torch.empty((N, L), dtype=torch.float64, device=dev)
    sums = torch.empty(N, dtype=torch.float64, device=dev) if stats else None
    prec = torch.empty(N, dtype=torch.float64, device=dev) if stats and W >= 8 else None
    err = torch.empty(1, dtype=torch.int64, device=dev)
    check(_lib.lib().fl_rule_rank_weights(fk._stream(rows), ptr(att), 1 if att.dtype == torch.float64 else 0, H, T, L,
                                          n, ptr(rows), N, W, ptr(row_head) if row_head is not None else None,
                                          int(identity), mode, ptr(rw), ptr(sums) if sums is not None else None,
                                          ptr(prec) if prec is not None else None, ptr(err)), "rule_rank_weights")
    code = int(err)
    if code == 1:
        raise IndexError("rule operator outside the attention's operator axis")
    if code == 2:
        raise IndexError("row head outside the attention batch")
    return rw, sums, prec


def _weights(attention, rows, identity, mode):
    dev = _device()
    att = _attention_tensor(attention, dev, False)
    r = _rows_tensor(rows, dev)
    if r.shape[0] == 0:
        return np.zeros((0, att.shape[2]), dtype=np.float64)
    return _annotate(att, r, None, identity, mode, stats=False)[0].cpu().numpy()


def _three_step_weights(attention, rows, identity):
    """Rank weights of 3-step attention by the closed form per body length
    (rules/extract.py:65-105)."""
    if np.asarray(attention).shape[0] != 3:
        raise ValueError("the closed form needs 3 steps")
    return _weights(attention, rows, identity, _CLOSED_FORM)


def collapsed_rule_weights(attention, rows, identity, maximum=False):
    """Rank weights by the dynamic program over identity placements, with
    sums or maxima (rules/extract.py:108-129)."""
    return _weights(attention, rows, identity, _DP_MAX if maximum else _DP_SUM)


def attention_rank_weights(attention, rows, identity):
    """The closed form for 3 steps, else the summing dynamic program
    (rules/extract.py:132-136)."""
    if np.asarray(attention).shape[0] == 3:
        return _three_step_weights(attention, rows, identity)
    return collapsed_rule_weights(attention, rows, identity)


def _fallback_scores_gpu(rw, sums):
    if FALLBACK_CHANNEL_AGGREGATION == "max":
        return rw.amax(dim=1)
    return sums


def fallback_rule_scores(rank_weights):
    """Per candidate the sum (or, with FALLBACK_CHANNEL_AGGREGATION "max",
    the maximum) of its channel weights (rules/extract.py:141-145)."""
    rw = torch.as_tensor(np.asarray(rank_weights, dtype=np.float64)).to(_device()).contiguous()
    if FALLBACK_CHANNEL_AGGREGATION == "max":
        return rw.amax(dim=1).cpu().numpy()
    out = torch.empty(rw.shape[0], dtype=torch.float64, device=rw.device)
    check(_lib.lib().fl_row_pairwise_sums(fk._stream(rw), ptr(rw), rw.shape[0], rw.shape[1], ptr(out)),
          "row_pairwise_sums")
    return out.cpu().numpy()


def _body_columns(rows, T):
    """Body operator p (1-based) of each row, -1 past its length."""
    return [torch.where(rows[:, 0] >= p, rows[:, p], torch.full_like(rows[:, 0], -1)) for p in range(1, T + 1)]


def _stable_order(keys, n, dev):
    """Permutation sorting by keys, given most significant first as
    (tensor, descending); ties keep input order."""
    perm = torch.arange(n, device=dev)
    for key, desc in reversed(keys):
        perm = perm[torch.sort(key[perm], descending=desc, stable=True).indices]
    return perm


def _select(rows, rw, sums, prec, minimum_positive_walks, T):
    """(selected, precision, rank weights, used_fallback) of one head's
    candidates, ordered (rules/extract.py:148-201); all on the GPU."""
    dev = rows.device
    N = rows.shape[0]
    picked = torch.nonzero(rows[:, -6] >= minimum_positive_walks).flatten()
    used_fallback = False
    if picked.numel() == 0 and N:
        used_fallback = True
        # Python's max over candidates by (score, body tuple): the first of the largest
        totals = _fallback_scores_gpu(rw, sums)
        keys = [(totals, True)] + [(c, True) for c in _body_columns(rows, T)]
        picked = _stable_order(keys, N, dev)[:1]
    sel, rws, sms, prs = rows[picked], rw[picked], sums[picked], prec[picked]
    keys = [(sel[:, -5], True), (sms, True)] + [(c, False) for c in _body_columns(sel, T)]
    order = _stable_order(keys, sel.shape[0], dev)
    return sel[order], prs[order], rws[order], used_fallback


def select_and_annotate_array(candidates, attention, identity, minimum_positive_walks):
    """Candidates with at least ``minimum_positive_walks`` positive walk
    hits (else the fallback's single best), their precision and rank
    weights, in output order (rules/extract.py:148-201)."""
    dev = _device()
    att = _attention_tensor(attention, dev, False)
    rows = _rows_tensor(candidates, dev)
    T = att.shape[1]
    if rows.shape[1] < max(8, 1 + T):
        raise ValueError("candidate rows need the body and the eight count columns")
    mode = _CLOSED_FORM if T == 3 else _DP_SUM
    rw, sums, prec = _annotate(att, rows, None, identity, mode)
    sel, pr, rws, fb = _select(rows, rw, sums, prec, minimum_positive_walks, T)
    return sel.cpu().numpy(), pr.cpu().numpy(), rws.cpu().numpy(), fb


def select_and_annotate_batch(candidates_list, attentions, identity, minimum_positive_walks):
    """select_and_annotate_array over the heads of one attention batch
    ([heads, steps, channels, operators]): one rank-weight launch over every
    head's candidates, then each head's selection on the GPU."""
    dev = _device()
    att = _attention_tensor(attentions, dev, True)
    H, T = att.shape[0], att.shape[1]
    if len(candidates_list) != H:
        raise ValueError("one candidate array per head")
    parts = [_rows_tensor(c, dev) for c in candidates_list]
    widths = {p.shape[1] for p in parts if p.shape[0]}
    if len(widths) > 1:
        raise ValueError("candidate arrays must have equal widths")
    W = widths.pop() if widths else 1 + T + 8
    if W < max(8, 1 + T):
        raise ValueError("candidate rows need the body and the eight count columns")
    counts = [p.shape[0] for p in parts]
    rows = torch.cat([p.reshape(-1, W) for p in parts]) if sum(counts) else torch.zeros((0, W), dtype=torch.int64,
                                                                                       device=dev)
    head = torch.repeat_interleave(torch.arange(H, device=dev), torch.tensor(counts, device=dev))
    mode = _CLOSED_FORM if T == 3 else _DP_SUM
    if rows.shape[0]:
        rw, sums, prec = _annotate(att, rows.contiguous(), head.contiguous(), identity, mode)
    else:
        rw = torch.zeros((0, att.shape[2]), dtype=torch.float64, device=dev)
        sums = prec = torch.zeros(0, dtype=torch.float64, device=dev)
    out, off = [], 0
    for c in counts:
        sl = slice(off, off + c)
        sel, pr, rws, fb = _select(rows[sl], rw[sl], sums[sl], prec[sl], minimum_positive_walks, T)
        out.append((sel.cpu().numpy(), pr.cpu().numpy(), rws.cpu().numpy(), fb))
        off += c
    return out


def output_lines(head, selected, precision, rank_weights):
    """Detailed rule rows of one head, CRLF-terminated, in FIELDS order
    (rules/extract.py:216-250)."""
    lines = []
    for row, p, weights in zip(selected, precision, rank_weights):
        length = int(row[0])
        body = " ".join(map(str, row[1:1 + length]))
        ranks = " ".join(f"{w:.17g}" for w in weights)
        cells = (head, body, length, f"{sum(weights):.17g}", row[-8], row[-7], row[-6], row[-5], row[-4], row[-3],
                 row[-2], row[-1], "flashlog-graph-guided-rule", ranks, f"{p:.17g}")
        lines.append("\t".join(map(str, cells)) + "\r\n")
    return lines


def output_rule_lines(head, selected, precision, rank_weights, operator_text=None):
    """Detailed rows and the rank-split scalar rows (one per channel with a
    positive weight, group_id = channel; SCALAR_FIELDS order) of one head
    (rules/extract.py:253-299).  operator_text maps operator ids to the
    body's text."""
    detailed, scalar = [], []
    head_text = str(head)
    for row, p, weights in zip(selected, precision, rank_weights):
        length = int(row[0])
        ops = row[1:1 + length]
        body = " ".join(map(str, ops)) if operator_text is None else " ".join(operator_text[o] for o in ops)
        texts = tuple(f"{w:.17g}" for w in weights)
        detailed.append(f"{head_text}\t{body}\t{length}\t{sum(weights):.17g}\t"
                        f"{row[-8]}\t{row[-7]}\t{row[-6]}\t{row[-5]}\t{row[-4]}\t{row[-3]}\t{row[-2]}\t{row[-1]}\t"
                        f"flashlog-graph-guided-rule\t{' '.join(texts)}\t{p:.17g}\r\n")
        prefix = f"{head_text}\t{body}\t{length}\t"
        for group, (w, text) in enumerate(zip(weights, texts)):
            if w > 0:
                scalar.append(f"{prefix}{text}\t{group}\tflashlog-rank-weighted-rule\r\n")
    return detailed, scalar
