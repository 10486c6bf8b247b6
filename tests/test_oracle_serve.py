"""The continuous-batching bookkeeping oracle (server/engine.py:522-620) on
hand-worked cases: every expected value below is worked out by hand from the
scenario, not recomputed with the oracle's formula."""

import torch

from oracle.serve import SlotState, block_tokens, tick_update

MASK, STOP, K, BL, NMAX, LMAX, D = 99, 98, 3, 4, 16, 40, 2


def make_state():
    xt = torch.full((6, NMAX), MASK, dtype=torch.int64)
    xt[3, 4:8] = torch.tensor([5, 6, 7, 8])  # slot 3 is committing the block at 4..8
    xt[4, 12:16] = torch.tensor([1, 2, 3, 4])
    st = SlotState(
        xt=xt,
        blk_start=torch.tensor([0, 0, 8, 4, 12, 0]),
        k_step=torch.tensor([0, 0, 1, 2, 1, 2]),
        cache_len=torch.tensor([30, 30, 30, 20, 36, 30]),
        n_speech=torch.tensor([16, 16, 16, 16, 16, 16]),
        is_commit=torch.tensor([False, False, False, True, True, False]),
        shift_ctx=torch.zeros(12, 1, D),
    )
    return st


def test_block_tokens_reads_each_slots_current_block():
    st = make_state()
    blk = block_tokens(st, 6, BL)
    assert blk[3].tolist() == [5, 6, 7, 8]
    assert blk[4].tolist() == [1, 2, 3, 4]
    assert blk[0].tolist() == [MASK] * 4


def test_tick_transitions():
    st = make_state()
    xt_blk = block_tokens(st, 6, BL)
    xt_new = torch.tensor([
        [10, MASK, 11, 12],   # 0: one mask left -> keep denoising
        [10, 11, 12, 13],     # 1: fully unmasked -> commit next tick
        [10, STOP, 11, 12],   # 2: EOS -> never commits
        [70, 71, 72, 73],     # 3: committing row -> the scorer's block is ignored
        [80, 81, 82, 83],     # 4: committing row at both clamps
        [MASK, MASK, 1, 2],   # 5: last step (k 2 -> 3 = K) -> commit even with masks
    ])
    hidden = torch.arange(12 * BL * D, dtype=torch.float32).view(12, BL, D)
    flags, xt_final = tick_update(st, 6, xt_blk, xt_new, hidden, n_branch=2, K=K, mask_id=MASK, stop_id=STOP,
                                  max_len=LMAX)
    # commit rows keep their block; denoise rows take the scorer's
    assert xt_final[3].tolist() == [5, 6, 7, 8]
    assert xt_final[4].tolist() == [1, 2, 3, 4]
    assert xt_final[0].tolist() == [10, MASK, 11, 12]
    assert st.xt[0, 0:4].tolist() == [10, MASK, 11, 12]
    assert st.xt[2, 8:12].tolist() == [10, STOP, 11, 12]
    # flags: commit, n_mask_after, hit_eos, k_step, blk_start, n_speech
    assert flags.tolist() == [
        [0, 1, 0, 1, 0, 16],
        [0, 0, 0, 1, 0, 16],
        [0, 0, 1, 2, 8, 16],
        [1, 0, 0, 0, 8, 16],     # blk_start 4 + 4
        [1, 0, 0, 0, 12, 16],    # blk_start 12 + 4 clamped to NMAX - BL = 12
        [0, 2, 0, 3, 0, 16],
    ]
    assert st.cache_len.tolist() == [30, 30, 30, 24, 36, 30]  # 36 + 4 clamped to LMAX - BL = 36
    assert st.is_commit.tolist() == [False, True, False, False, False, True]
    # shift context of the committing slots (3, 4) = each row's last hidden position
    for row in (6, 7, 8, 9):
        assert torch.equal(st.shift_ctx[row, 0], hidden[row, BL - 1])
    assert st.shift_ctx[:6].abs().sum() == 0 and st.shift_ctx[10:].abs().sum() == 0


def test_only_first_n_slots_move():
    st = make_state()
    before = st.clone()
    xt_blk = block_tokens(st, 2, BL)
    tick_update(st, 2, xt_blk, xt_blk.clone(), torch.zeros(4, BL, D), n_branch=2, K=K, mask_id=MASK,
                stop_id=STOP, max_len=LMAX)
    for name in ("blk_start", "k_step", "cache_len", "is_commit"):
        assert torch.equal(getattr(st, name)[2:], getattr(before, name)[2:])
    assert torch.equal(st.xt[2:], before.xt[2:])
