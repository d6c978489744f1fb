"""The work list of the transposed backward (host logic, CPU): every non-zero of every row of A^T in exactly one
segment, one slot -1 segment per row starting at its first non-zero, the later segments' slots numbered
contiguously per row and listed in the row's split entry, longest segments first."""

from __future__ import annotations

import numpy as np
import pytest
import torch


@pytest.mark.parametrize("seg", [64, 128, 256])
def test_work_list_covers_every_non_zero_once(seg):
    from chessfly.brain import backward_work
    rng = np.random.default_rng(seg)
    lens = np.minimum(rng.lognormal(np.log(40), 1.2, 500).astype(np.int64), 3000)
    lens[[3, 77, 499]] = [0, 1000, seg]
    crow = torch.as_tensor(np.concatenate([[0], np.cumsum(lens)]))
    items, splits, n_slots = backward_work(crow.to(torch.int32), seg)
    items, splits = items.numpy().astype(np.int64), splits.numpy().astype(np.int64)
    assert items.shape[1] == 4 and splits.shape[1] == 4
    assert np.all(np.diff(items[:, 2]) <= 0)                       # longest first
    covered = np.zeros(int(lens.sum()), np.int64)
    firsts = np.zeros(len(lens), np.int64)
    slots_of = {}
    for row, off, count, slot in items:
        assert 0 <= count <= seg and 0 <= off and off + count <= lens[row]
        covered[crow[row] + off:crow[row] + off + count] += 1
        if slot < 0:
            assert off == 0
            firsts[row] += 1
        else:
            assert off > 0 and count > 0
            slots_of.setdefault(int(row), []).append((int(off), int(slot)))
    assert np.all(covered == 1) and np.all(firsts == 1)
    assert n_slots == sum(len(v) for v in slots_of.values())
    assert sorted(s for v in slots_of.values() for _, s in v) == list(range(n_slots))
    assert sorted(int(r) for r in splits[:, 0]) == sorted(slots_of)
    for row, first, count, zero in splits:
        segs = sorted(slots_of[int(row)])                           # by offset: slots follow the row's order
        assert zero == 0 and count == len(segs) == -(-lens[row] // seg) - 1
        assert [s for _, s in segs] == list(range(first, first + count))


def test_work_list_rejects_partial_blocks():
    from chessfly.brain import backward_work
    with pytest.raises(ValueError):
        backward_work(torch.tensor([0, 10], dtype=torch.int32), 100)
