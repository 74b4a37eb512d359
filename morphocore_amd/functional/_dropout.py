"""Weight dropout of the dilation and erosion functionals (reference: functional/dilation.py:78-87,
functional/erosion.py:78-87).

The reference draws ``rand_like(w) > p``, then walks the (out, in) channel pairs in order and, for
each pair left without a surviving tap, draws one ``randint(0, taps, (1,))`` on the default CPU
generator and keeps that tap; on a GPU every pair's ``.any()`` is a host synchronisation. Here the
pairs without a survivor are found in one pass and their taps drawn in one ``randint`` of as many
values, in the same pair order: the CPU generator produces the same values for one call of n draws as
for n calls of one, so a seeded run keeps exactly the reference's taps, with one host synchronisation.
The kept taps are set on the mask itself by their (out, in, row, column) indices, so a weight that is
not contiguous (a permuted view, whose ``rand_like`` keeps its strides) gets them too.
"""
import torch


def dropout_keep(w: torch.Tensor, p: float) -> torch.Tensor:
    """Boolean mask of the taps of ``w`` that survive weight dropout with probability ``p``; at least
    one tap of every (out, in) pair (dims 0 and 1) survives."""
    keep = torch.rand_like(w) > p
    pairs = w.shape[0] * w.shape[1]
    taps = w[0, 0].numel() if pairs else 0
    dead = ~keep.reshape(pairs, taps).any(dim=1)  # read only: reshape may copy a non-contiguous mask
    n_dead = int(dead.sum())  # the one host synchronisation
    if n_dead:
        tap = torch.randint(0, taps, (n_dead,)).to(keep.device)
        pair = dead.nonzero().squeeze(1)
        index = (pair // w.shape[1], pair % w.shape[1])
        if w.dim() > 2:
            index = index + tuple(torch.unravel_index(tap, tuple(w.shape[2:])))
        keep[index] = True
    return keep


def drop_weights(w: torch.Tensor, p: float) -> torch.Tensor:
    """``w`` with the taps dropout removes set to -inf (they never win a dilation, nor an erosion, which
    subtracts them), as the reference's dilation / erosion do in training (dilation.py:78-87)."""
    keep = dropout_keep(w, p)
    return torch.where(keep, w, torch.tensor(-float('inf'), device=w.device, dtype=w.dtype))
