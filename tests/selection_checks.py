"""Checks of a selection that hold row by row without an oracle run.

``closed_form_counts`` is the valid-count rule of the top-k expansion
(``ops/csrc/topk.cu:152-162`` of the reference); ``logical_invariants``
checks every row of a logical selection at once on the device.
"""

import torch


def closed_form_counts(positions, seq_lens, token_to_req, ratio, k):
    """``count = min(min((pos+1)//R, seq//R, k) * R + (pos+1) mod R, seq)``."""
    p1 = positions.long() + 1
    seq = seq_lens.long()[token_to_req.long()]
    complete = torch.minimum(torch.minimum(p1 // ratio, seq // ratio), torch.full_like(p1, k))
    return torch.minimum(complete * ratio + p1 % ratio, seq)


def logical_invariants(idx, positions, seq_lens, token_to_req, visible, ratio, k):
    """Every row of a logical selection (on the device, all rows at once):
    valid entries are exactly the closed-form prefix; the block part is runs
    of R consecutive tokens of strictly ascending visible blocks; the tail is
    the visible incomplete block's tokens; every token is <= the position."""
    rows, width = idx.shape
    counts = closed_form_counts(positions, seq_lens, token_to_req, ratio, k)
    col = torch.arange(width, device=idx.device)
    assert torch.equal(idx >= 0, col[None, :] < counts[:, None]), "valid prefix"
    p1 = positions.long() + 1
    complete = torch.minimum(torch.minimum(p1 // ratio, seq_lens.long()[token_to_req.long()]
                                           // ratio), torch.full_like(p1, k))
    in_blocks = col[None, :] < (complete * ratio)[:, None]
    t = idx.long()
    assert bool(((t % ratio == col % ratio) | ~in_blocks).all()), "page-aligned runs"
    blocks = t[:, :k * ratio].view(rows, k, ratio)
    first = blocks[:, :, 0]
    assert bool(((blocks - first[..., None]) == torch.arange(ratio, device=idx.device))
                [in_blocks[:, :k * ratio].view(rows, k, ratio)].all()), "runs of R tokens"
    ranked = torch.arange(k, device=idx.device)[None, :] < complete[:, None]
    step = first[:, 1:] - first[:, :-1]
    assert bool((step > 0)[ranked[:, 1:]].all()), "blocks strictly ascending"
    assert bool(((first // ratio) < visible.long()[:, None])[ranked].all()), "blocks visible"
    tail_start = (p1 // ratio) * ratio
    in_tail = (idx >= 0) & ~in_blocks
    tail_want = tail_start[:, None] + (col[None, :] - (complete * ratio)[:, None])
    assert torch.equal(t[in_tail], tail_want[in_tail]), "causal tail"
    assert bool((t <= positions.long()[:, None]).all()), "causal"
