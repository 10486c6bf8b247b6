"""Pins of the page-math oracle (oracle/pages.py) on the CPU.

* ``page_write_indices`` against the identity-table closed form of
  engines/flashinfer.py:318-344 (``page = r*P + pos//16``, ``slot = pos%16``)
  for one start and for per-row starts, and against a brute-force position
  map on random tables;
* ``plan`` against the closed form of engines/flashinfer.py:346-411
  (``qo_indptr = b*bl``, ``kv_indptr`` = running sum of ``ceil(kv/16)``,
  ``last_page_len = kv % 16 or 16``) and against the native planner's
  coverage of the same rows;
* ``pool_write`` / ``pool_gather`` on position-coded K and V: every element
  lands where the layout's closed form puts it (plane 0 token-major
  ``t*64 + d``, plane 1 transposed ``d*16 + t``), nothing else is touched,
  and the gather returns exactly what was written, for tiles of 1-3 pages.
"""

import numpy as np
import pytest
import torch

from oracle import pages as OP
from yapd_amd import kernels

PS = 16


def identity_table(B, P):
    return np.arange(B * P, dtype=np.int64).reshape(B, P)


@pytest.mark.parametrize("cs", [0, 5, 16, 31, 100])
@pytest.mark.parametrize("bl", [1, 16, 32])
def test_write_indices_identity_closed_form_int_start(cs, bl):
    B, P = 3, 16
    pages, slots = OP.page_write_indices(identity_table(B, P), cs, bl)
    pos = np.arange(cs, cs + bl)
    exp_pages = np.concatenate([b * P + pos // PS for b in range(B)])
    exp_slots = np.tile(pos % PS, B)
    assert np.array_equal(pages, exp_pages) and np.array_equal(slots, exp_slots)


def test_write_indices_identity_closed_form_list_starts():
    B, P, bl = 4, 20, 32
    starts = [0, 15, 17, 250]
    pages, slots = OP.page_write_indices(identity_table(B, P), starts, bl)
    exp_p = np.concatenate([b * P + np.arange(cs, cs + bl) // PS for b, cs in enumerate(starts)])
    exp_s = np.concatenate([np.arange(cs, cs + bl) % PS for cs in starts])
    assert np.array_equal(pages, exp_p) and np.array_equal(slots, exp_s)
    # an int start equals the same start repeated in a list
    a = OP.page_write_indices(identity_table(B, P), 17, bl)
    b = OP.page_write_indices(identity_table(B, P), [17] * B, bl)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))


def test_write_indices_brute_force_random_tables():
    rng = np.random.default_rng(0)
    for trial in range(20):
        B, P = int(rng.integers(1, 6)), int(rng.integers(2, 12))
        n_pages = B * P + int(rng.integers(0, 9))
        table = rng.permutation(n_pages)[: B * P].reshape(B, P)
        bl = int(rng.integers(1, 33))
        starts = [int(rng.integers(0, P * PS - bl + 1)) for _ in range(B)]
        # brute force: enumerate every (page, slot) of the table and look positions up
        where = {}
        for r in range(B):
            for j in range(P):
                for t in range(PS):
                    where[(r, j * PS + t)] = (int(table[r][j]), t)
        pages, slots = OP.page_write_indices(table, starts, bl)
        exp = [where[(r, cs + j)] for r, cs in enumerate(starts) for j in range(bl)]
        assert [(int(p), int(s)) for p, s in zip(pages, slots)] == exp
        # distinct tokens of one call never share a (page, slot)
        assert len(set(exp)) == len(exp)


@pytest.mark.parametrize("kv", [[1, 15, 16, 17, 32, 33, 288], 48])
def test_plan_identity_closed_form(kv):
    B, P, bl = 7, 20, 32
    qo, kvi, idx, last = OP.plan(identity_table(B, P), kv, bl)
    kv = [kv] * B if isinstance(kv, int) else kv
    pu = [-(-k // PS) for k in kv]
    assert qo.tolist() == [b * bl for b in range(B + 1)]
    assert kvi.tolist() == [sum(pu[:b]) for b in range(B + 1)]
    assert idx.tolist() == [b * P + j for b in range(B) for j in range(pu[b])]
    assert last.tolist() == [k % PS if k % PS else PS for k in kv]
    # kv_len a multiple of 16: a full last page (not 0)
    assert all(l == 16 for k, l in zip(kv, last) if k % 16 == 0)
    assert all(1 <= l <= PS for l in last)


def test_plan_random_table_matches_native_coverage():
    """The oracle's per-row page list equals the set of pages the native
    planner's work items touch for the same kv lengths (any split)."""
    rng = np.random.default_rng(1)
    B, P = 9, 140
    table = rng.permutation(B * P + 50)[: B * P].reshape(B, P)
    kv = [1, 16, 17, 500, 1024, 1025, 2047, 2048, 2222]
    qo, kvi, idx, last = OP.plan(table, kv, 16)
    for target, min_split in ((1024, 1024), (4096, 32)):
        work, merge, n_slots = kernels.attn_plan(kv, target_items=target, min_split_keys=min_split)
        for r in range(B):
            touched = set()
            for row, kb, ke, _ in work.tolist():
                if row == r:
                    touched.update(int(table[r][p]) for p in range(kb // PS, (ke - 1) // PS + 1))
            assert touched == set(idx[kvi[r]: kvi[r + 1]].tolist())
            n_full = kvi[r + 1] - kvi[r] - 1
            assert n_full * PS + last[r] == kv[r]


@pytest.mark.parametrize("n_pages_tile", [1, 2, 3])
def test_pool_write_gather_round_trip_position_coded(n_pages_tile):
    H, hd = 4, 64
    rng = np.random.default_rng(n_pages_tile)
    B, P = 3, 6
    n_pages = B * P + 5
    table = rng.permutation(n_pages)[: B * P].reshape(B, P)
    bl = n_pages_tile * PS - (3 if n_pages_tile > 1 else 0)  # ragged last page
    starts = [0, 7, 2 * PS + 9]
    N = B * bl
    # K carries (token, dim) in two fields and V (token, head): any misplaced
    # element shows up as a wrong code
    tok = torch.arange(N).view(-1, 1, 1).expand(N, H, hd)
    hh = torch.arange(H).view(1, -1, 1).expand(N, H, hd)
    dd = torch.arange(hd).view(1, 1, -1).expand(N, H, hd)
    k = (tok * 4096 + hh * 64 + dd).float()           # exact in fp32
    v = -(tok * 4096 + hh * 64 + dd).float() - 1.0
    sentinel = 1e9
    pool = torch.full((n_pages, 2, H, PS * hd), sentinel, dtype=torch.float32)
    OP.pool_write(pool, table, starts, k, v)
    # closed form of the layout for every written token
    written = set()
    for r, cs in enumerate(starts):
        for j in range(bl):
            n, pos = r * bl + j, cs + j
            p, t = int(table[r][pos // PS]), pos % PS
            for h in range(H):
                for d in (0, 1, 31, 63):
                    assert pool[p, 0, h, t * hd + d].item() == k[n, h, d].item()
                    assert pool[p, 1, h, d * PS + t].item() == v[n, h, d].item()
            written.add((p, t))
    # every other slot is untouched
    for p in range(n_pages):
        for t in range(PS):
            if (p, t) not in written:
                assert (pool[p, 0].view(H, PS, hd)[:, t] == sentinel).all()
                assert (pool[p, 1].view(H, hd, PS)[:, :, t] == sentinel).all()
    # gather returns exactly the written K and V (both planes) for each row
    for r, cs in enumerate(starts):
        K, V = OP.pool_gather(pool, table[r], cs + bl)
        assert torch.equal(K[cs:], k[r * bl:(r + 1) * bl])
        assert torch.equal(V[cs:], v[r * bl:(r + 1) * bl])
        assert (K[:cs] == sentinel).all() and (V[:cs] == sentinel).all()
