"""The native attention planner (host code, no GPU): every key of every row is
covered exactly once, split items are whole 32-key chunks, merge records
match the split items, and items come longest first."""

import numpy as np
import pytest

from yapd_amd import kernels
from yapd_amd.synthetic import log_uniform_lengths


@pytest.mark.parametrize("target", [1, 8, 64, 1024])
def test_plan_covers_every_key_once(target):
    kv = [L + 16 for L in log_uniform_lengths(50, 64, 2048, seed=target)] + [1, 31, 32, 33]
    work, merge, n_slots = kernels.attn_plan(kv, target_items=target, min_split_keys=128)
    cover = {r: [] for r in range(len(kv))}
    slots = set()
    for row, kb, ke, slot in work.tolist():
        assert 0 <= kb < ke <= kv[row]
        cover[row].append((kb, ke))
        if slot >= 0:
            assert kb % 32 == 0 and slot not in slots
            slots.add(slot)
    for r, spans in cover.items():
        spans.sort()
        assert spans[0][0] == 0 and spans[-1][1] == kv[r]
        for (a, b), (c, d) in zip(spans, spans[1:]):
            assert b == c
    assert len(slots) == n_slots
    for row, first, cnt in merge.tolist():
        assert cnt >= 2 and len(cover[row]) == cnt
        owned = sorted(s for (rw, kb, ke, s) in work.tolist() if rw == row)
        assert owned == list(range(first, first + cnt))
    lens = [ke - kb for (_, kb, ke, _) in work.tolist()]
    assert lens == sorted(lens, reverse=True)


def test_plan_no_split_when_enough_rows():
    kv = [400] * 600
    work, merge, n_slots = kernels.attn_plan(kv, target_items=512)
    assert n_slots == 0 and len(merge) == 0 and len(work) == 600


def test_plan_rejects_bad_lengths():
    with pytest.raises(ValueError):
        kernels.attn_plan([10, 0, 5])
    with pytest.raises(ValueError):
        kernels.attn_plan([10], min_split_keys=16)


def test_host_uploads_keep_values_dtype_and_shape():
    """``to_device_async`` (plan, row-list and index uploads) converts lists, numpy arrays and
    numpy slices exactly; on the CPU it is a plain conversion (the pinned, stream-ordered copy is
    the GPU branch, exercised by every engine test)."""
    import numpy as np
    import torch
    from yapd_amd.paged import AttnPlan, to_device_async
    assert torch.equal(to_device_async([3, 1, 2], torch.long, torch.device("cpu")), torch.tensor([3, 1, 2]))
    arr = np.arange(12, dtype=np.int32).reshape(3, 4)
    t = to_device_async(arr, torch.int32, "cpu")
    assert t.dtype == torch.int32 and torch.equal(t, torch.from_numpy(arr))
    t = to_device_async(arr[1, :3], torch.int64, "cpu")
    assert t.dtype == torch.int64 and t.tolist() == [4, 5, 6]
    plan = AttnPlan([700, 40, 1600], 16, 16, torch.device("cpu"))
    assert plan.work.dtype == torch.int32 and plan.work.shape[1] == 4
    assert plan.kv_len.tolist() == [700, 40, 1600]
